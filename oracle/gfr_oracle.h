/* CPU oracle for the EXL3 MoE-expert path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's scalar algorithm (glm-flash-rs, src/experts.rs:12-135 and the
 * formulas of native/exl3.cu / native/grouping.cu). Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or the timed CPU baseline; the product path
 * (libgfr_moe.so) never links or calls it.
 *
 * fp16 / bf16 values travel as their raw uint16 bit patterns.
 */
#ifndef GFR_ORACLE_H
#define GFR_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

uint16_t gfro_f32_to_f16(float x);          /* IEEE binary16, round to nearest even (half 2.7 from_f32) */
float gfro_f16_to_f32(uint16_t h);
float gfro_hf(float x);                     /* experts.rs:22-24  fp32 -> fp16 -> fp32 */
float gfro_bf(float x);                     /* experts.rs:19-21  bf16 round-to-nearest-even, bit form */
uint16_t gfro_f32_to_bf16(float x);         /* upper half of gfro_bf(x) */
float gfro_bf16_to_f32(uint16_t b);

uint16_t gfro_codebook(uint32_t s);         /* experts.rs:43-46 == exl3.cu:21-30 (mcg2), fp16 bits */
void gfro_codebook_table(uint16_t* out);    /* all 65536 states */
float gfro_codebook_sum(uint32_t s);        /* the two halves summed, unrounded (the decode GEMV's weight) */
int gfro_tile_words(int bits);              /* 32-bit words in a 16x16 tile: 256 * bits / 32 */
uint32_t gfro_state(const uint32_t* tile, int bits, int p);   /* experts.rs:58-64 generalised to K bits */
void gfro_tile_pos(int p, int* row, int* col);                /* experts.rs:65-69 */
/* experts.rs:47-74: trellis words [kin/16][n/16][tile_words] -> row-major fp16 bits [kin][n] */
void gfro_unpack(const uint32_t* words, int kin, int n, int bits, uint16_t* w);
void gfro_unpack_f32(const uint32_t* words, int kin, int n, int bits, float* w);
void gfro_unpack_f32_sum(const uint32_t* words, int kin, int n, int bits, float* w);  /* unrounded weights */

void gfro_had(float* x, long n);            /* experts.rs:25-42: unnormalised FWHT per 128-block */
/* experts.rs:75-96: y[n] = sum_j x[j] w[j][n], K split into sk * warps contiguous ranges summed in order */
void gfro_matmul(const float* x, const float* w, int k, int n, int sk, int warps, float* y);

/* exl3.cu:224-241 rot_in for one (pair, matrix): out = fp16(had(bf16 x * suh) * HAD) */
void gfro_rot(const uint16_t* x_bf16, const uint16_t* suh, int k, uint16_t* out);
/* exl3.cu:260-296 gateup epilogue on already-summed partials g,u [n] (modified in place) -> xd fp16 [n] */
void gfro_gateup_epilogue(float* g, float* u, const uint16_t* svh_g, const uint16_t* svh_u,
                          const uint16_t* suh_d, int n, float limit, uint16_t* xd);
/* exl3.cu:300-321 down epilogue on summed partials z [d] (in place) -> y fp32 [d] */
void gfro_down_epilogue(float* z, const uint16_t* svh_d, int d, float* y);
void gfro_rot_rows(const uint16_t* x_bf16, long x_stride, const int32_t* rows, int nrows, const uint16_t* suh, int k,
                   uint16_t* out);
void gfro_gateup_epilogue_rows(float* g, float* u, const uint16_t* svh_g, const uint16_t* svh_u,
                               const uint16_t* suh_d, int nrows, int n, float limit, uint16_t* xd);
void gfro_down_epilogue_rows(float* z, const uint16_t* svh_d, int nrows, int d, float* y);

/* One expert on one row (experts.rs:113-135, reference_first, generalised to the shape): decoded weights
 * wg, wu [D][N], wd [N][D] as fp32 (gfro_unpack_f32), per-expert scale vectors. sk_gu / sk_d / warps give the
 * fixed summation order (the decode path: 4 / 1 / 4; the prefill path: 1 / 1 / 1). Writes y [D] and, if
 * xd != NULL, the fp16 down-projection input [N]. */
void gfro_expert_row(const uint16_t* x_bf16, int D, int N, const float* wg, const float* wu, const float* wd,
                     const uint16_t* suh_g, const uint16_t* suh_u, const uint16_t* suh_d,
                     const uint16_t* svh_g, const uint16_t* svh_u, const uint16_t* svh_d,
                     int sk_gu, int sk_d, int warps, float limit, float* y, uint16_t* xd);

/* Single EXL3 linear: y = svh * had(W^T xh) * HAD, xh = fp16(had(x * suh) * HAD),
 * x fp16. */
void gfro_linear(const uint16_t* x_f16, int kin, int n, const float* w, const uint16_t* suh,
                 const uint16_t* svh, float* y);

/* grouping.cu:1-100 / grouping.rs:141-192: stable token->expert bucketing.
 * picks [rows][slots] expert ids in [0, E); count = distinct experts; ids[u] ascending; members[u*maxm + i] =
 * r*32 + slot (first slot of e in row r), rows ascending, -1 tails; members rows u in [count, E) all -1.
 * Returns 0, or -1 on a precondition failure (id out of range, rows > maxm). */
int gfro_group(const int32_t* picks, int rows, int slots, int E, int maxm, int32_t* ids, int32_t* count,
               int32_t* members);

/* Router of the benchmark configs (softmax top-k, renormalised; source of the reference's Triton topk is
 * absent): picks[r][0..topk) by descending logit (ties: lower id), picks[r][topk] = shared_id, weights the
 * renormalised softmax of the picked logits, weight 1 for the shared slot. */
void gfro_route(const float* logits, int rows, int E, int topk, int shared_id, int32_t* picks, float* weights);
void gfro_route_biased(const float* logits, const float* bias, float scale, int rows, int E, int topk, int shared_id,
                       int32_t* picks, float* weights);
/* out[r][n] = sum over slots in order of weights[r][s] * y[r*slots+s][n] */
void gfro_combine(const float* y, const float* weights, int rows, int slots, int D, float* out);

/* The FP8 shared expert (moe.rs:132-167) as the reference's scalar oracle states it.
 * front.rs:173-182 fp8: an e4m3 byte -> f32 (exponent 0: m * 2^-9; else (1 + m / 8) * 2^(e - 7); 0x7f -> 480 as
 * there, although the format calls it NaN). */
float gfro_fp8(uint8_t v);
/* front.rs:190-217 reference_mm_at: y[n] = sum over sk contiguous K slices (in order) of (the slice's sequential fp32
 * sum of x[j] * fp8(w[n][j])) * bf16 scale[n]; round != 0: y rounded to bf16 (as a float). w [n][k] bytes. */
void gfro_fp8_matmul(const float* x, const uint8_t* w, const uint16_t* scale_bf16, int k, int n, int sk, int round,
                     float* y);
/* prefill.cu:7-17 f8_b16_copy: out[n][k] = bf16_rn(fp8(w[n][k]) * bf16 scale[n]) (bf16 bits; exponent 15 mantissa 7
 * -> NaN there) */
void gfro_fp8_b16_copy(const uint8_t* w, const uint16_t* scale_bf16, int n, int k, uint16_t* out);
/* front.rs:669-675: act[j] = bf(bf(g / (1 + exp(-g))) * u), g = min(gu[j], limit), u = clamp(gu[inter + j], +-limit) */
void gfro_shared_swiglu(const float* gu, int inter, float limit, float* act);

/* The CPU baseline of bench.py: decode + fp32 matvec of the given experts for one token, timed inside C
 * (experts.rs:43-96 path: unpack, codebook, fixed-order matmul). Returns seconds; writes y [n_exp][D]. */
double gfro_baseline_decode(const uint16_t* x_bf16, int D, int N, int bits, int n_exp, const int32_t* experts,
                            const uint32_t* gt, const uint32_t* ut, const uint32_t* dt,
                            const uint16_t* suh_g, const uint16_t* suh_u, const uint16_t* suh_d,
                            const uint16_t* svh_g, const uint16_t* svh_u, const uint16_t* svh_d, float* y);

#ifdef __cplusplus
}
#endif
#endif
