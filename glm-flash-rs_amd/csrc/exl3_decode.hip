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
    h2_t d[2][2][4];
    decode_lane<K>(w, prev, d);
    if (!ok) return;
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int l = 0; l < 4; ++l) {
                const int row = kt * 16 + 2 * l + 8 * h, col = nt * 16 + i + 8 * c;
                const uint32_t v = h2_bits(d[c][h][l]);
                out[(size_t)row * n + col] = (uint16_t)v;
                out[(size_t)(row + 1) * n + col] = (uint16_t)(v >> 16);
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
    const uint32_t packed = (uint32_t)f32_to_f16(v[0] * HAD_SCALE) | ((uint32_t)f32_to_f16(v[1] * HAD_SCALE) << 16);
    *reinterpret_cast<uint32_t*>(o) = packed;
}

// Grouped trellis GEMV. Program (distinct expert u, 128-column block cb, mat * SK + split): the members of expert
// uids[u] (rows of X, RB at a time) times W_q[mat] over k tiles [split * NW * KTW, (split + 1) * NW * KTW) for the
// block's 128 columns; wave w owns k tiles split * NW * KTW + w * KTW + [0, KTW).
// Z[((mat * SK + split) * P + pair) * N + n]. MATS = 2 (gate + up) or 1 (down): separate kernels for the profiler.
template <int K, int KTW, int NW, int RB, int MATS>
__global__ void __launch_bounds__(NW * 64) gemv_kernel(
    const uint16_t* __restrict__ X0, const uint16_t* __restrict__ X1, const uint32_t* __restrict__ T0,
    const uint32_t* __restrict__ T1, const int* __restrict__ uids, const int* __restrict__ ucount,
    const int* __restrict__ members, float* __restrict__ Z, int Kin, int N, int P, int SK, int maxm, int slots,
    int E) {
    constexpr int KC = NW * KTW;                 // k tiles a workgroup
    constexpr int MAXM = 64;                     // member rows a workgroup can hold (the engine's max_rows bound)
    __shared__ int rows_sh[MAXM];
    __shared__ int cnt_sh;
    __shared__ __attribute__((aligned(16))) uint16_t xs[RB][KC * 16];
    __shared__ float red[NW][RB][128];

    const int u = blockIdx.x;
    if (u >= ucount[0]) return;
    const int e = uids[u];
    if (e >= E) return;                          // not an EXL3 expert
    const int cb = blockIdx.y, split = blockIdx.z % SK, mat = MATS == 1 ? 0 : blockIdx.z / SK;
    const uint16_t* __restrict__ X = mat ? X1 : X0;
    const uint32_t* __restrict__ T = mat ? T1 : T0;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, t = lane >> 3, i = lane & 7;
    const int KT = Kin >> 4, NT = N >> 4;
    const int kt0 = split * KC + wave * KTW;

    // this wave's trellis words, all KTW k tiles issued before anything else
    uint32_t wr[KTW][K];
    {
        const uint32_t* src = T + (((size_t)e * KT + kt0) * NT + cb * 8 + t) * (8 * K) + i * K;
#pragma unroll
        for (int kk = 0; kk < KTW; ++kk) load_words<K>(src + (size_t)kk * NT * (8 * K), wr[kk]);
    }

    if (tid == 0) cnt_sh = 0;
    __syncthreads();
    for (int m = tid; m < maxm && m < MAXM; m += NW * 64) {
        const int code = members[(size_t)u * maxm + m];
        rows_sh[m] = code >= 0 ? (code >> 5) * slots + (code & 31) : -1;
        if (code >= 0) atomicMax(&cnt_sh, m + 1);   // members come first
    }
    __syncthreads();
    const int cnt = cnt_sh;

    for (int r0 = 0; r0 < cnt; r0 += RB) {
        const int nr = cnt - r0 < RB ? cnt - r0 : RB;
        // the member rows' k range into LDS (16-byte chunks)
        for (int c = tid; c < nr * KC * 2; c += NW * 64) {
            const int m = c / (KC * 2), q = c % (KC * 2);
            const uint16_t* src = X + (size_t)rows_sh[r0 + m] * Kin + (size_t)split * KC * 16 + q * 8;
            *reinterpret_cast<uint4*>(&xs[m][q * 8]) = *reinterpret_cast<const uint4*>(src);
        }
        __syncthreads();
        float acc[RB][2];
#pragma unroll
        for (int m = 0; m < RB; ++m) acc[m][0] = acc[m][1] = 0.f;
#pragma unroll
        for (int kk = 0; kk < KTW; ++kk) {
            const uint32_t prev = prev_word(wr[kk][K - 1], i);
            h2_t d[2][2][4];
            decode_lane<K>(wr[kk], prev, d);
            const int kx = (wave * KTW + kk) * 16;
#pragma unroll
            for (int m = 0; m < RB; ++m) {
                if (m < nr) {
                    const uint4 xa = *reinterpret_cast<const uint4*>(&xs[m][kx]);
                    const uint4 xb = *reinterpret_cast<const uint4*>(&xs[m][kx + 8]);
                    const uint32_t xl[2][4] = {{xa.x, xa.y, xa.z, xa.w}, {xb.x, xb.y, xb.z, xb.w}};
#pragma unroll
                    for (int l = 0; l < 4; ++l)
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const h2_t xv = bits_h2(xl[h][l]);
                            acc[m][0] = __builtin_amdgcn_fdot2(d[0][h][l], xv, acc[m][0], false);
                            acc[m][1] = __builtin_amdgcn_fdot2(d[1][h][l], xv, acc[m][1], false);
                        }
                }
            }
        }
#pragma unroll
        for (int m = 0; m < RB; ++m)
            if (m < nr) {
                red[wave][m][16 * t + i] = acc[m][0];
                red[wave][m][16 * t + i + 8] = acc[m][1];
            }
        __syncthreads();
        for (int idx = tid; idx < nr * 128; idx += NW * 64) {
            const int m = idx >> 7, col = idx & 127;
            float s = red[0][m][col];
#pragma unroll
            for (int w = 1; w < NW; ++w) s += red[w][m][col];
            Z[((size_t)(mat * SK + split) * P + rows_sh[r0 + m]) * N + cb * 128 + col] = s;
        }
        __syncthreads();                             // xs / red are rewritten by the next chunk
    }
}

// gateup epilogue (exl3.cu:260-296): ordered split sums of gate and up, rotation, svh scales, GLM's limited SwiGLU
// with its bf16 roundings, suh_d scale, rotation -> xd fp16. One wave a (pair, 128-column block).
__global__ void __launch_bounds__(64) gateup_epilogue_kernel(const float* __restrict__ Z, const int* __restrict__ pick,
                                                              const uint16_t* __restrict__ svh_g,
                                                              const uint16_t* __restrict__ svh_u,
                                                              const uint16_t* __restrict__ suh_d,
                                                              uint16_t* __restrict__ xd, int P, int N, int SK,
                                                              int slots, int exl3_slots, float limit) {
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
    const uint32_t packed = (uint32_t)f32_to_f16(v[0] * HAD_SCALE) | ((uint32_t)f32_to_f16(v[1] * HAD_SCALE) << 16);
    *reinterpret_cast<uint32_t*>(xd + (size_t)p * N + n) = packed;
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

constexpr int GEMV_NW = 4, GEMV_RB = 8;

static int gemv_ktw(int Kin) {
    const int KT = Kin / 16;
    return KT % (GEMV_NW * 4) == 0 ? 4 : KT % (GEMV_NW * 2) == 0 ? 2 : 1;
}

int gemv_splits(int Kin) { return Kin / 16 / (GEMV_NW * gemv_ktw(Kin)); }

template <int K, int MATS>
static void gemv_dispatch(int ktw, dim3 grid, hipStream_t s, const uint16_t* X0, const uint16_t* X1,
                          const uint32_t* T0, const uint32_t* T1, const int* uids, const int* ucount,
                          const int* members, float* Z, int Kin, int N, int P, int SK, int maxm, int slots, int E) {
    if (ktw == 4)
        gemv_kernel<K, 4, GEMV_NW, GEMV_RB, MATS><<<grid, GEMV_NW * 64, 0, s>>>(X0, X1, T0, T1, uids, ucount, members, Z,
                                                                          Kin, N, P, SK, maxm, slots, E);
    else if (ktw == 2)
        gemv_kernel<K, 2, GEMV_NW, GEMV_RB, MATS><<<grid, GEMV_NW * 64, 0, s>>>(X0, X1, T0, T1, uids, ucount, members, Z,
                                                                          Kin, N, P, SK, maxm, slots, E);
    else
        gemv_kernel<K, 1, GEMV_NW, GEMV_RB, MATS><<<grid, GEMV_NW * 64, 0, s>>>(X0, X1, T0, T1, uids, ucount, members, Z,
                                                                          Kin, N, P, SK, maxm, slots, E);
}

hipError_t launch_gemv(hipStream_t s, const uint16_t* X0, const uint16_t* X1, const uint32_t* T0, const uint32_t* T1,
                       const int* uids, const int* ucount, const int* members, float* Z, int Kin, int N, int P,
                       int maxm, int slots, int E, int bits, int mats, int maxu) {
    const int ktw = gemv_ktw(Kin), SK = gemv_splits(Kin);
    const dim3 grid(maxu, N / 128, mats * SK);
    if (mats == 2) {
        switch (bits) {
            case 2: gemv_dispatch<2, 2>(ktw, grid, s, X0, X1, T0, T1, uids, ucount, members, Z, Kin, N, P, SK, maxm, slots, E); break;
            case 3: gemv_dispatch<3, 2>(ktw, grid, s, X0, X1, T0, T1, uids, ucount, members, Z, Kin, N, P, SK, maxm, slots, E); break;
            case 4: gemv_dispatch<4, 2>(ktw, grid, s, X0, X1, T0, T1, uids, ucount, members, Z, Kin, N, P, SK, maxm, slots, E); break;
            case 5: gemv_dispatch<5, 2>(ktw, grid, s, X0, X1, T0, T1, uids, ucount, members, Z, Kin, N, P, SK, maxm, slots, E); break;
            default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
    }
    switch (bits) {
        case 2: gemv_dispatch<2, 1>(ktw, grid, s, X0, X1, T0, T1, uids, ucount, members, Z, Kin, N, P, SK, maxm, slots, E); break;
        case 3: gemv_dispatch<3, 1>(ktw, grid, s, X0, X1, T0, T1, uids, ucount, members, Z, Kin, N, P, SK, maxm, slots, E); break;
        case 4: gemv_dispatch<4, 1>(ktw, grid, s, X0, X1, T0, T1, uids, ucount, members, Z, Kin, N, P, SK, maxm, slots, E); break;
        case 5: gemv_dispatch<5, 1>(ktw, grid, s, X0, X1, T0, T1, uids, ucount, members, Z, Kin, N, P, SK, maxm, slots, E); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gateup_epilogue(hipStream_t s, const float* Z, const int* pick, const uint16_t* svh_g,
                                  const uint16_t* svh_u, const uint16_t* suh_d, uint16_t* xd, int P, int N, int SK,
                                  int slots, int exl3_slots, float limit) {
    gateup_epilogue_kernel<<<dim3(P, N / 128), 64, 0, s>>>(Z, pick, svh_g, svh_u, suh_d, xd, P, N, SK, slots,
                                                           exl3_slots, limit);
    return hipGetLastError();
}

hipError_t launch_down_epilogue(hipStream_t s, const float* Z, const int* pick, const uint16_t* svh_d, float* y,
                                int P, int D, int SK, int slots, int exl3_slots) {
    down_epilogue_kernel<<<dim3(P, D / 128), 64, 0, s>>>(Z, pick, svh_d, y, P, D, SK, slots, exl3_slots);
    return hipGetLastError();
}

}  // namespace gfr
