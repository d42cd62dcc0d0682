/* CPU oracle for the EXL3 MoE-expert path -- TEST INFRASTRUCTURE ONLY (tests/, smoke(), bench.py's
 * cpu_baseline leg). Never linked into libgfr_moe.so.
 *
 * Every function restates the reference glm-flash-rs (paths relative to its repository root) and cites the
 * lines it follows. Compiled with -ffp-contract=off so that a*b+c stays two roundings, as in the Rust
 * reference (rustc never contracts).
 */
#include "gfr_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

static const float HAD = 0.08838834764831845f; /* experts.rs:11 (0.088_388_346), exl3.cu:18 */

static uint32_t fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bitsf(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16 round-to-nearest-even, the conversion of the `half` crate (Cargo.lock:456) and __float2half_rn */
uint16_t gfro_f32_to_f16(float f) {
    uint32_t x = fbits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);      /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                          /* below 2^-14: subnormal or zero */
        if (ax <= 0x33000000u) return (uint16_t)sign;                 /* <= 2^-25 (a tie) rounds to 0 */
        uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t sh = 126u - e, q = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t h = (ax - 0x38000000u) >> 13, rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float gfro_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return bitsf(sign);
        float v = (float)m * 5.9604644775390625e-08f;                 /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) return bitsf(sign | 0x7f800000u | (m << 13));
    return bitsf(sign | ((e + 112u) << 23) | (m << 13));
}

float gfro_hf(float x) { return gfro_f16_to_f32(gfro_f32_to_f16(x)); }   /* experts.rs:22-24 */

/* experts.rs:19-21, bit for bit (no NaN special case, as there) */
float gfro_bf(float x) {
    uint32_t b = fbits(x);
    return bitsf((b + 0x7fffu + ((b >> 16) & 1u)) & 0xffff0000u);
}
uint16_t gfro_f32_to_bf16(float x) { return (uint16_t)(fbits(gfro_bf(x)) >> 16); }
float gfro_bf16_to_f32(uint16_t b) { return bitsf((uint32_t)b << 16); }

/* experts.rs:43-46 (== exl3.cu:21-30 mcg2 for one state): the two halves of the scrambled state summed and
 * rounded to fp16 */
uint16_t gfro_codebook(uint32_t s) {
    uint32_t x = ((s * 0xcbac1fedu) & 0x8fff8fffu) ^ 0x3b603b60u;
    return gfro_f32_to_f16(gfro_f16_to_f32((uint16_t)x) + gfro_f16_to_f32((uint16_t)(x >> 16)));
}

/* The same two halves summed in fp32 and not rounded: the weight as this library's decode GEMV multiplies it (one
 * v_dot2_f32_f16 of both halves against the activation). Exact: both halves are fp16 of magnitude 2^-3 .. 2, so the
 * sum needs at most 16 significant bits. gfro_codebook(s) is this value rounded to fp16. */
float gfro_codebook_sum(uint32_t s) {
    uint32_t x = ((s * 0xcbac1fedu) & 0x8fff8fffu) ^ 0x3b603b60u;
    return gfro_f16_to_f32((uint16_t)x) + gfro_f16_to_f32((uint16_t)(x >> 16));
}

void gfro_codebook_table(uint16_t* out) {
    for (uint32_t s = 0; s < 65536u; ++s) out[s] = gfro_codebook(s);
}

int gfro_tile_words(int bits) { return 8 * bits; }

/* experts.rs:58-64: the 16-bit window of the tile's circular bitstream (words in order, MSB first within a
 * word) that ends at bit (p + 1) * bits. The reference fixes bits = 4 (first = p*4 + 4 + 1024 - 16); the tile
 * length 256 * bits generalises the 1024. */
uint32_t gfro_state(const uint32_t* tile, int bits, int p) {
    const long B = 256L * bits, W = 8L * bits;
    const long last = (long)(p + 1) * bits + B, first = last - 16;
    const long i0 = (first / 32) % W, i1 = ((last - 1) / 32) % W;
    const long shift = ((last - 1) / 32 + 1) * 32 - last;
    return (uint32_t)(((((uint64_t)tile[i0]) << 32) | (uint64_t)tile[i1]) >> shift) & 0xffffu;
}

/* experts.rs:65-69: value p of a tile sits at (row, col) of the 16 x 16 block (row = k, col = n) */
void gfro_tile_pos(int p, int* row, int* col) {
    const int lane = p / 8, j = p % 8;
    *row = 2 * (lane % 4) + (j & 1) + 8 * ((j >> 1) & 1);
    *col = lane / 4 + 8 * (j >> 2);
}

/* experts.rs:47-74: tile (kt, nt) starts at word (kt * n/16 + nt) * tile_words */
void gfro_unpack(const uint32_t* words, int kin, int n, int bits, uint16_t* w) {
    const int TW = gfro_tile_words(bits);
    for (int kt = 0; kt < kin / 16; ++kt)
        for (int nt = 0; nt < n / 16; ++nt) {
            const uint32_t* tile = words + ((size_t)kt * (n / 16) + nt) * TW;
            for (int p = 0; p < 256; ++p) {
                int row, col;
                gfro_tile_pos(p, &row, &col);
                w[(size_t)(kt * 16 + row) * n + nt * 16 + col] = gfro_codebook(gfro_state(tile, bits, p));
            }
        }
}

/* gfro_unpack with the unrounded sums of gfro_codebook_sum (the decode GEMV's weights) */
void gfro_unpack_f32_sum(const uint32_t* words, int kin, int n, int bits, float* w) {
    const int TW = gfro_tile_words(bits);
    for (int kt = 0; kt < kin / 16; ++kt)
        for (int nt = 0; nt < n / 16; ++nt) {
            const uint32_t* tile = words + ((size_t)kt * (n / 16) + nt) * TW;
            for (int p = 0; p < 256; ++p) {
                int row, col;
                gfro_tile_pos(p, &row, &col);
                w[(size_t)(kt * 16 + row) * n + nt * 16 + col] = gfro_codebook_sum(gfro_state(tile, bits, p));
            }
        }
}

void gfro_unpack_f32(const uint32_t* words, int kin, int n, int bits, float* w) {
    uint16_t* h = (uint16_t*)malloc((size_t)kin * n * 2);
    gfro_unpack(words, kin, n, bits, h);
    for (size_t i = 0; i < (size_t)kin * n; ++i) w[i] = gfro_f16_to_f32(h[i]);
    free(h);
}

/* experts.rs:25-42: in-place unnormalised Walsh-Hadamard transform of each full 128-block, butterflies at
 * strides 1, 2, ..., 64, (a + b, a - b) */
void gfro_had(float* x, long n) {
    for (long b0 = 0; b0 + 128 <= n; b0 += 128) {
        float* block = x + b0;
        for (int stride = 1; stride < 128; stride *= 2)
            for (int base = 0; base < 128; base += 2 * stride)
                for (int j = 0; j < stride; ++j) {
                    const float a = block[base + j], b = block[base + j + stride];
                    block[base + j] = a + b;
                    block[base + j + stride] = a - b;
                }
    }
}

/* experts.rs:75-96: the decode kernels' fixed order -- K in sk splits of `warps` contiguous ranges, each range
 * summed in ascending k, the ranges of a split added left to right, the splits added in order */
void gfro_matmul(const float* x, const float* w, int k, int n, int sk, int warps, float* y) {
    float* acc = (float*)malloc(sizeof(float) * (size_t)warps);
    const int len = k / (sk * warps);
    for (int col = 0; col < n; ++col) {
        float sum = 0.f;
        for (int split = 0; split < sk; ++split) {
            for (int wp = 0; wp < warps; ++wp) {
                const int begin = (split * warps + wp) * len;
                float a = 0.f;
                for (int j = begin; j < begin + len; ++j) a += x[j] * w[(size_t)j * n + col];
                acc[wp] = a;
            }
            float partial = acc[0];
            for (int wp = 1; wp < warps; ++wp) partial += acc[wp];
            sum += partial;
        }
        y[col] = sum;
    }
    free(acc);
}

/* exl3.cu:224-241 (and experts.rs:117-118): Xh = fp16(had(bf16 x * fp16 suh) * HAD) */
void gfro_rot(const uint16_t* x_bf16, const uint16_t* suh, int k, uint16_t* out) {
    float* v = (float*)malloc(sizeof(float) * (size_t)k);
    for (int i = 0; i < k; ++i) v[i] = gfro_bf16_to_f32(x_bf16[i]) * gfro_f16_to_f32(suh[i]);
    gfro_had(v, k);
    for (int i = 0; i < k; ++i) out[i] = gfro_f32_to_f16(v[i] * HAD);
    free(v);
}

/* exl3.cu:260-296 (experts.rs:120-138): after the ordered split sums */
void gfro_gateup_epilogue(float* g, float* u, const uint16_t* svh_g, const uint16_t* svh_u,
                          const uint16_t* suh_d, int n, float limit, uint16_t* xd) {
    gfro_had(g, n);
    gfro_had(u, n);
    for (int i = 0; i < n; ++i) {
        const float gg = fminf(gfro_bf(g[i] * HAD * gfro_f16_to_f32(svh_g[i])), limit);
        const float uu = fminf(fmaxf(gfro_bf(u[i] * HAD * gfro_f16_to_f32(svh_u[i])), -limit), limit);
        const float act = gfro_bf(gfro_bf(gg / (1.f + expf(-gg))) * uu);
        g[i] = act * gfro_f16_to_f32(suh_d[i]);
    }
    gfro_had(g, n);
    for (int i = 0; i < n; ++i) xd[i] = gfro_f32_to_f16(g[i] * HAD);
}

/* exl3.cu:300-321 (experts.rs:141-145) */
void gfro_down_epilogue(float* z, const uint16_t* svh_d, int d, float* y) {
    gfro_had(z, d);
    for (int i = 0; i < d; ++i) y[i] = z[i] * HAD * gfro_f16_to_f32(svh_d[i]);
}

/* Row batches of the three per-row steps above, for checking whole windows: each is exactly a loop of the single-row
 * function over the rows (tests/test_oracle.py checks that), nothing else. rot: row r of out = gfro_rot of input row
 * rows[r] of x [*][x_stride] with scale vector suh. The epilogues: row r of g / u / z in place, as gfro_gateup_epilogue
 * / gfro_down_epilogue. */
void gfro_rot_rows(const uint16_t* x_bf16, long x_stride, const int32_t* rows, int nrows, const uint16_t* suh, int k,
                   uint16_t* out) {
    for (int r = 0; r < nrows; ++r) gfro_rot(x_bf16 + (size_t)rows[r] * x_stride, suh, k, out + (size_t)r * k);
}

void gfro_gateup_epilogue_rows(float* g, float* u, const uint16_t* svh_g, const uint16_t* svh_u,
                               const uint16_t* suh_d, int nrows, int n, float limit, uint16_t* xd) {
    for (int r = 0; r < nrows; ++r)
        gfro_gateup_epilogue(g + (size_t)r * n, u + (size_t)r * n, svh_g, svh_u, suh_d, n, limit, xd + (size_t)r * n);
}

void gfro_down_epilogue_rows(float* z, const uint16_t* svh_d, int nrows, int d, float* y) {
    for (int r = 0; r < nrows; ++r) gfro_down_epilogue(z + (size_t)r * d, svh_d, d, y + (size_t)r * d);
}

/* experts.rs:113-146 reference_first, at any shape and split order */
void gfro_expert_row(const uint16_t* x_bf16, int D, int N, const float* wg, const float* wu, const float* wd,
                     const uint16_t* suh_g, const uint16_t* suh_u, const uint16_t* suh_d,
                     const uint16_t* svh_g, const uint16_t* svh_u, const uint16_t* svh_d,
                     int sk_gu, int sk_d, int warps, float limit, float* y, uint16_t* xd) {
    uint16_t* xh = (uint16_t*)malloc(2 * (size_t)(D > N ? D : N));
    float* xf = (float*)malloc(sizeof(float) * (size_t)(D > N ? D : N));
    float* g = (float*)malloc(sizeof(float) * (size_t)N);
    float* u = (float*)malloc(sizeof(float) * (size_t)N);
    uint16_t* xdl = (uint16_t*)malloc(2 * (size_t)N);
    float* z = (float*)malloc(sizeof(float) * (size_t)D);
    gfro_rot(x_bf16, suh_g, D, xh);
    for (int i = 0; i < D; ++i) xf[i] = gfro_f16_to_f32(xh[i]);
    gfro_matmul(xf, wg, D, N, sk_gu, warps, g);
    gfro_rot(x_bf16, suh_u, D, xh);
    for (int i = 0; i < D; ++i) xf[i] = gfro_f16_to_f32(xh[i]);
    gfro_matmul(xf, wu, D, N, sk_gu, warps, u);
    gfro_gateup_epilogue(g, u, svh_g, svh_u, suh_d, N, limit, xdl);
    for (int i = 0; i < N; ++i) xf[i] = gfro_f16_to_f32(xdl[i]);
    gfro_matmul(xf, wd, N, D, sk_d, warps, z);
    gfro_down_epilogue(z, svh_d, D, y);
    if (xd) memcpy(xd, xdl, 2 * (size_t)N);
    free(xh); free(xf); free(g); free(u); free(xdl); free(z);
}

/* A single EXL3 linear (the benchmark's config 1): rot_in's formula on an fp16 token, one GEMV, the down
 * epilogue's formula (exl3.cu:224-241, 300-321) */
void gfro_linear(const uint16_t* x_f16, int kin, int n, const float* w, const uint16_t* suh,
                 const uint16_t* svh, float* y) {
    float* v = (float*)malloc(sizeof(float) * (size_t)kin);
    float* z = (float*)malloc(sizeof(float) * (size_t)n);
    for (int i = 0; i < kin; ++i) v[i] = gfro_f16_to_f32(x_f16[i]) * gfro_f16_to_f32(suh[i]);
    gfro_had(v, kin);
    for (int i = 0; i < kin; ++i) v[i] = gfro_hf(v[i] * HAD);
    gfro_matmul(v, w, kin, n, 1, 1, z);
    gfro_down_epilogue(z, svh, n, y);
    free(v); free(z);
}

/* grouping.cu:17-64 (bitmap path) == grouping.cu:67-100 (small path) == grouping.rs:141-160 host oracle for
 * distinct picks: a (row, expert) is recorded once, with the first slot that holds the expert */
int gfro_group(const int32_t* picks, int rows, int slots, int E, int maxm, int32_t* ids, int32_t* count,
               int32_t* members) {
    if (rows < 0 || rows > maxm || slots < 1 || slots > 32) return -1;
    for (long i = 0; i < (long)rows * slots; ++i)
        if (picks[i] < 0 || picks[i] >= E) return -1;
    int* n = (int*)calloc((size_t)E, sizeof(int));
    for (int r = 0; r < rows; ++r)
        for (int s = 0; s < slots; ++s) {
            int first = 1;
            for (int q = 0; q < s; ++q) first &= picks[r * slots + q] != picks[r * slots + s];
            if (first) n[picks[r * slots + s]]++;
        }
    int c = 0;
    for (int e = 0; e < E; ++e)
        if (n[e]) ids[c++] = e;
    *count = c;
    for (long i = 0; i < (long)E * maxm; ++i) members[i] = -1;
    for (int u = 0; u < c; ++u) {
        const int e = ids[u];
        int off = 0;
        for (int r = 0; r < rows; ++r)
            for (int s = 0; s < slots; ++s)
                if (picks[r * slots + s] == e) {
                    members[(long)u * maxm + off++] = r * 32 + s;
                    break;
                }
    }
    free(n);
    return 0;
}

void gfro_route(const float* logits, int rows, int E, int topk, int shared_id, int32_t* picks, float* weights) {
    const int slots = topk + 1;
    char* used = (char*)malloc((size_t)E);
    for (int r = 0; r < rows; ++r) {
        const float* l = logits + (size_t)r * E;
        memset(used, 0, (size_t)E);
        for (int s = 0; s < topk; ++s) {
            int best = -1;
            for (int e = 0; e < E; ++e)
                if (!used[e] && (best < 0 || l[e] > l[best])) best = e;
            used[best] = 1;
            picks[r * slots + s] = best;
        }
        const float m = l[picks[r * slots]];
        float sum = 0.f;
        for (int s = 0; s < topk; ++s) {
            weights[r * slots + s] = expf(l[picks[r * slots + s]] - m);
            sum += weights[r * slots + s];
        }
        for (int s = 0; s < topk; ++s) weights[r * slots + s] = weights[r * slots + s] / sum;
        picks[r * slots + topk] = shared_id;
        weights[r * slots + topk] = 1.f;
    }
    free(used);
}

/* GLM's gate for the reference's `topk` call (moe.rs:89-99: logits, bias, picks, weights, 2.5; its Triton source is
 * absent): the published DeepSeek-V3 / GLM-4.5 "noaux" gating. score = sigmoid(logit) in float; top-k by
 * score + bias (ties: lower id); weight = score / (sum of the picked scores in slot order + 1e-20) * scale; the shared
 * expert last with weight 1. PARITY UNPINNED against the reference (binary-only kernel). */
void gfro_route_biased(const float* logits, const float* bias, float scale, int rows, int E, int topk, int shared_id,
                       int32_t* picks, float* weights) {
    const int slots = topk + 1;
    char* used = (char*)malloc((size_t)E);
    float* sc = (float*)malloc((size_t)E * sizeof(float));
    float* ch = (float*)malloc((size_t)E * sizeof(float));
    for (int r = 0; r < rows; ++r) {
        const float* l = logits + (size_t)r * E;
        for (int e = 0; e < E; ++e) {
            sc[e] = 1.f / (1.f + expf(-l[e]));
            ch[e] = sc[e] + bias[e];
        }
        memset(used, 0, (size_t)E);
        for (int s = 0; s < topk; ++s) {
            int best = -1;
            for (int e = 0; e < E; ++e)
                if (!used[e] && (best < 0 || ch[e] > ch[best])) best = e;
            used[best] = 1;
            picks[r * slots + s] = best;
        }
        float sum = 0.f;
        for (int s = 0; s < topk; ++s) sum += sc[picks[r * slots + s]];
        for (int s = 0; s < topk; ++s) weights[r * slots + s] = sc[picks[r * slots + s]] / (sum + 1e-20f) * scale;
        picks[r * slots + topk] = shared_id;
        weights[r * slots + topk] = 1.f;
    }
    free(used);
    free(sc);
    free(ch);
}

void gfro_combine(const float* y, const float* weights, int rows, int slots, int D, float* out) {
    for (int r = 0; r < rows; ++r)
        for (int n = 0; n < D; ++n) {
            float acc = 0.f;
            for (int s = 0; s < slots; ++s) acc += weights[r * slots + s] * y[((size_t)r * slots + s) * D + n];
            out[(size_t)r * D + n] = acc;
        }
}

static double now_s(void) {
    struct timespec t;
    clock_gettime(CLOCK_MONOTONIC, &t);
    return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

double gfro_baseline_decode(const uint16_t* x_bf16, int D, int N, int bits, int n_exp, const int32_t* experts,
                            const uint32_t* gt, const uint32_t* ut, const uint32_t* dt,
                            const uint16_t* suh_g, const uint16_t* suh_u, const uint16_t* suh_d,
                            const uint16_t* svh_g, const uint16_t* svh_u, const uint16_t* svh_d, float* y) {
    const size_t tiles = (size_t)(D / 16) * (N / 16), TW = (size_t)gfro_tile_words(bits);
    float* wg = (float*)malloc(sizeof(float) * (size_t)D * N);
    float* wu = (float*)malloc(sizeof(float) * (size_t)D * N);
    float* wd = (float*)malloc(sizeof(float) * (size_t)D * N);
    const double t0 = now_s();
    for (int i = 0; i < n_exp; ++i) {
        const size_t e = (size_t)experts[i];
        gfro_unpack_f32(gt + e * tiles * TW, D, N, bits, wg);
        gfro_unpack_f32(ut + e * tiles * TW, D, N, bits, wu);
        gfro_unpack_f32(dt + e * tiles * TW, N, D, bits, wd);
        gfro_expert_row(x_bf16, D, N, wg, wu, wd, suh_g + e * D, suh_u + e * D, suh_d + e * N, svh_g + e * N,
                        svh_u + e * N, svh_d + e * D, 4, 1, 4, 10.f, y + (size_t)i * D, NULL);
    }
    const double t = now_s() - t0;
    free(wg); free(wu); free(wd);
    return t;
}

/* ---- the FP8 shared expert (moe.rs:132-167) ---- */
float gfro_fp8(uint8_t v) {
    const int e = (v >> 3) & 15, m = v & 7;
    const float sign = (v & 128) ? -1.f : 1.f;
    if (e == 0) return sign * (float)m * ldexpf(1.f, -9);
    return sign * (1.f + (float)m / 8.f) * ldexpf(1.f, e - 7);
}

void gfro_fp8_matmul(const float* x, const uint8_t* w, const uint16_t* scale_bf16, int k, int n, int sk, int round,
                     float* y) {
    for (int r = 0; r < n; ++r) {
        const float s = gfro_bf16_to_f32(scale_bf16[r]);
        float sum = 0.f;
        for (int part = 0; part < sk; ++part) {
            float acc = 0.f;
            const long j0 = (long)part * k / sk, j1 = (long)(part + 1) * k / sk;
            for (long j = j0; j < j1; ++j) acc += x[j] * gfro_fp8(w[(size_t)r * k + j]);
            const float partial = acc * s;
            sum = part == 0 ? partial : sum + partial;
        }
        y[r] = round ? gfro_bf(sum) : sum;
    }
}

void gfro_shared_swiglu(const float* gu, int inter, float limit, float* act) {
    for (int j = 0; j < inter; ++j) {
        const float g = fminf(gu[j], limit);
        const float u = fminf(fmaxf(gu[inter + j], -limit), limit);
        act[j] = gfro_bf(gfro_bf(g / (1.f + expf(-g))) * u);
    }
}

void gfro_fp8_b16_copy(const uint8_t* w, const uint16_t* scale_bf16, int n, int k, uint16_t* out) {
    for (int r = 0; r < n; ++r) {
        const float s = gfro_bf16_to_f32(scale_bf16[r]);
        for (int j = 0; j < k; ++j) {
            const uint8_t b = w[(size_t)r * k + j];
            const int e = (b >> 3) & 15, m = b & 7;
            float x = e == 0 ? (float)m * 0.001953125f : ldexpf((float)(8 + m), e - 10);
            if (e == 15 && m == 7) x = NAN;
            if (b & 128) x = -x;
            out[(size_t)r * k + j] = gfro_f32_to_bf16(x * s);
        }
    }
}
