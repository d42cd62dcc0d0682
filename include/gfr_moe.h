/* gfr_moe -- MI355X (gfx950) EXL3 MoE-expert path behind a C ABI.
 *
 * Drop-in for the expert-dispatch surface of glm-flash-rs (paths relative to the reference repository):
 *   Grouping            src/grouping.rs:12-112        -> gfr_grouping_*
 *   ExpertGpu           src/experts.rs:365-564        -> gfr_experts_*       (decode / verify windows)
 *   FastExperts         src/fast_experts.rs:27-208    -> gfr_fast_experts_*  (prefill chunks)
 *   Moe::run_prefetched src/moe.rs:66-182             -> gfr_moe_*           (router .. combine)
 * The reference binds its kernels through the CUDA driver (src/cuda.rs); a Rust caller binds these functions with
 * `extern "C"` declarations of the prototypes below instead.
 *
 * Conventions (src/cuda.rs:102-123, experts.rs:461-464):
 *   - every function returns 0 on success, a negative GFR_E* code when a precondition fails, or a positive
 *     hipError_t; gfr_last_error() gives the thread's last message;
 *   - pointers are device addresses, fp16 / bf16 data travel as uint16_t bit patterns;
 *   - engines allocate their scratch once at create (zeroed); run functions never allocate, free or synchronise,
 *     are ordered on the caller's stream and can be captured into a HIP graph;
 *   - one host thread per engine; calls that overlap on one engine race on its scratch.
 */
#ifndef GFR_MOE_H
#define GFR_MOE_H
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GFR_OK 0
#define GFR_EINVAL (-1)   /* argument outside the engine's bounds (the reference's ensure!) */
#define GFR_ENOMEM (-2)
#define GFR_EUNSUPPORTED (-3)

/* One layer's EXL3 expert tensors, the reference's weights.layers[L].moe.experts.{gt,ut,dt,suh_*,svh_*}
 * (experts.rs:146-156, prepared.rs:369-377), generalised to any shape and bit width:
 *   gt, ut  [experts][hidden/16][inter/16][8*bits] uint32   (gate, up:  hidden -> inter)
 *   dt      [experts][inter/16][hidden/16][8*bits] uint32   (down:      inter -> hidden)
 *   suh_g, suh_u [experts][hidden], suh_d, svh_g, svh_u [experts][inter], svh_d [experts][hidden]   fp16
 * `experts` counts every EXL3 expert, the shared one included when it is EXL3 (then it is the last index). */
typedef struct gfr_exl3_experts {
    int experts;
    int hidden;
    int inter;
    int bits; /* 2, 3, 4 or 5 */
    const uint32_t* gt;
    const uint32_t* ut;
    const uint32_t* dt;
    const uint16_t* suh_g;
    const uint16_t* suh_u;
    const uint16_t* suh_d;
    const uint16_t* svh_g;
    const uint16_t* svh_u;
    const uint16_t* svh_d;
} gfr_exl3_experts;

const char* gfr_last_error(void);
/* Library version string. */
const char* gfr_version(void);

/* ---- Grouping (grouping.rs:12-112) ---------------------------------------------------------------------------
 * picks [rows][slots] int32 expert ids in [0, experts). After run: *count = distinct experts, ids[u] ascending,
 * members[u * max_rows + i] = r * 32 + slot (rows ascending, the first slot of the expert in the row), -1 padded;
 * members rows u in [count, experts) all -1. slots <= 32. */
typedef struct gfr_grouping gfr_grouping;
int gfr_grouping_create(gfr_grouping** out, int experts, int slots, int max_rows);  /* Grouping::new  :29-50 */
int gfr_grouping_run(gfr_grouping* g, hipStream_t stream, const int32_t* picks, int rows); /* Grouping::run :51-112 */
int32_t* gfr_grouping_ids(const gfr_grouping* g);      /* [experts]            (Grouping.ids)     */
int32_t* gfr_grouping_count(const gfr_grouping* g);    /* [1]                  (Grouping.count)   */
int32_t* gfr_grouping_members(const gfr_grouping* g);  /* [experts][max_rows]  (Grouping.members) */
int gfr_grouping_destroy(gfr_grouping* g);

/* ---- Decode / verify experts (ExpertGpu, experts.rs:365-564) -------------------------------------------------
 * slots = picks per row (routed + shared); the first exl3_slots slots are EXL3 experts (the reference:
 * slots - 1, its shared expert is FP8; the benchmark configs: slots, the shared expert is EXL3).
 * run_rows: input [rows][input_stride] bf16; picks [rows][slots]; ids / count / members from a gfr_grouping with
 * member stride maxm. Output gfr_experts_y: [rows * slots][hidden] fp32 (pairs with slot >= exl3_slots untouched).
 * Bounds: 0 < rows <= max_rows, rows <= maxm <= max_rows, max_rows <= 64.
 * Arithmetic: each weight enters as its two fp16 codebook halves times the activation, summed in fp32 (the
 * reference first rounds their sum to an fp16 weight); outputs stay within 1e-2 relative of the reference's
 * (about 1.2e-3 measured). The same holds for the bs = 1 layer of gfr_moe, gfr_linear and gfr_exl3_grouped_gemv. */
typedef struct gfr_experts gfr_experts;
int gfr_experts_create(gfr_experts** out, int hidden, int inter, int slots, int exl3_slots, int max_rows);
int gfr_experts_run_rows(gfr_experts* ex, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                         int input_stride, const int32_t* picks, const int32_t* ids, const int32_t* count,
                         const int32_t* members, int rows, int maxm);  /* ExpertGpu::run_rows :447-563 */
float* gfr_experts_y(const gfr_experts* ex);
uint16_t* gfr_experts_xd(const gfr_experts* ex);   /* [rows * slots][inter] fp16, the down projection's input */
int gfr_experts_destroy(gfr_experts* ex);

/* ---- Prefill experts (FastExperts, fast_experts.rs:27-208) ---------------------------------------------------
 * Same inputs as run_rows for a chunk of up to max_rows rows; the grouped GEMM runs on fp16 MFMA with one
 * full-K accumulation chain per output. shared_x != 0 asserts suh_g == suh_u (one rotated copy of the rows).
 * Output gfr_fast_experts_output: [rows * slots][hidden] fp32; gfr_fast_experts_xd [rows * slots][inter] fp16. */
typedef struct gfr_fast_experts gfr_fast_experts;
int gfr_fast_experts_create(gfr_fast_experts** out, int hidden, int inter, int slots, int exl3_slots, int experts,
                            int max_rows);                                          /* FastExperts::new :43-64 */
int gfr_fast_experts_run(gfr_fast_experts* fx, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                         int input_stride, const int32_t* picks, const int32_t* ids, const int32_t* count,
                         const int32_t* members, int rows, int maxm, int shared_x);  /* FastExperts::run :91-208 */
float* gfr_fast_experts_output(const gfr_fast_experts* fx);
uint16_t* gfr_fast_experts_xd(const gfr_fast_experts* fx);
/* Parity probe, no reference counterpart (the reference keeps rot_in's output internal, exl3.cu:224-241): the rotated
 * input rows of the last run, [rows * slots][hidden] fp16, matrix 0 (gate, or both when shared_x) or 1 (up); each
 * 16-value k tile stored in pair order: u16 2m holds x[m + 8], 2m + 1 holds x[m] (m = 0..7). Null for mat not 0 or 1. */
uint16_t* gfr_fast_experts_rotated(const gfr_fast_experts* fx, int mat);
int gfr_fast_experts_destroy(gfr_fast_experts* fx);

/* ---- One MoE layer (Moe::run_prefetched, moe.rs:66-182) ------------------------------------------------------
 * logits [rows][routed] fp32 router logits -> softmax top-k (renormalised) + the shared expert (id `routed`,
 * weight 1) -> grouping -> experts (decode path for rows <= decode_rows, prefill path above) -> combine ->
 * output [rows][hidden] fp32, the slots added in order.
 * gfr_moe_create: the shared expert is EXL3 (the benchmark configs); the weights hold routed + 1 experts.
 * gfr_moe_create_shared with shared_exl3 = 0: the reference's layout, whose shared expert is FP8 and runs outside the
 * EXL3 path (moe.rs:132-167); the weights hold the routed experts only, and the caller's shared-expert output enters
 * the combine as the last slot (gfr_moe_run_shared: out = sum of the routed slots' weighted outputs + shared, the
 * reference's combine(y, shared, weights, out), moe.rs:171-181). */
typedef struct gfr_moe gfr_moe;
int gfr_moe_create(gfr_moe** out, int hidden, int inter, int routed, int topk, int max_rows);  /* Moe::new :23-64 */
int gfr_moe_create_shared(gfr_moe** out, int hidden, int inter, int routed, int topk, int max_rows, int shared_exl3);
int gfr_moe_run(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                const float* logits, int rows);                                 /* Moe::run_prefetched :66-182 */
/* shared [rows][shared_stride] fp32: the shared expert's output (a layer made with shared_exl3 = 0 only);
 * shared_stride a multiple of 4 and shared 16-byte aligned (read 16 bytes at a time). */
int gfr_moe_run_shared(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                       const float* logits, const float* shared, int shared_stride, int rows);
/* The routed branch of shared_expert.rs Branch::run (:60-78): the caller forks its own shared expert onto another
 * stream and records shared_ready there once `shared` is written; the routed experts run on `stream` and only the
 * combine (the last launch) waits for the event, so the two branches overlap. Same result as gfr_moe_run_shared. */
int gfr_moe_run_shared_branch(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                              const float* logits, const float* shared, int shared_stride, int rows,
                              hipEvent_t shared_ready);
/* The whole layer from the hidden rows: router logits (gfr_router_logits, the reference's router_part + router_sum,
 * moe.rs:77-87) into the layer's own buffer, then gfr_moe_run_shared (shared may be NULL: no shared term, or an
 * EXL3 shared expert). router_weight [routed][hidden] bf16. */
int gfr_moe_run_router(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                       const uint16_t* router_weight, const float* shared, int shared_stride, int rows);
float* gfr_moe_output(const gfr_moe* m);
int32_t* gfr_moe_picks(const gfr_moe* m);        /* [rows][topk + 1] */
float* gfr_moe_weights(const gfr_moe* m);        /* [rows][topk + 1] */
/* Parity probe, no reference counterpart (as gfr_fast_experts_rotated): the rotated input rows of the last run on
 * the prefill engine (windows above decode_rows), [rows * (topk + 1)][hidden] fp16 in the same pair order, matrix 0
 * (gate) or 1 (up). Windows of at most 256 rows rotate them in the route + group launch. Null for mat not 0 or 1. */
uint16_t* gfr_moe_rotated(const gfr_moe* m, int mat);
/* Windows of at most decode_rows rows run the decode engine (default 4, at most 64), larger ones the prefill engine.
 * rows == 1 runs three launches: gate/up GEMV (router and input rotation fused), down GEMV (gate/up epilogue fused),
 * sum of the down parts + combine. */
int gfr_moe_set_decode_rows(gfr_moe* m, int decode_rows);
/* No counterpart in the reference: for callers that cannot allocate device memory (code under HIP graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). One token through the bs = 1 layer of gfr_moe_run (the
 * router's softmax gate over `routed` experts, top-k, the EXL3 shared expert last: w holds routed + 1 experts), the
 * same kernels and arithmetic, with every scratch buffer in a fixed 8 MiB device array of the library (one a GPU,
 * held until the process ends); a shape whose scratch exceeds it (about 2 slots x hidden x inter / 32 bytes plus
 * 50 slots x hidden bytes) returns GFR_EINVAL. Allocates nothing. The array keeps the last call's contents; calls that
 * overlap on one GPU race on it. out [hidden] fp32; picks / weights [topk + 1] copies of the routing (may be NULL). */
int gfr_moe_token_static(hipStream_t stream, const gfr_exl3_experts* w, int routed, int topk, const uint16_t* input,
                         const float* logits, float* out, int32_t* picks, float* weights);
/* The layer's router gate: bias == NULL (default) the softmax gate of gfr_route_topk; else GLM's gate of
 * gfr_route_topk_biased with this bias [routed] (device, fp32; must outlive the runs) and scale (2.5 for GLM). */
int gfr_moe_set_router(gfr_moe* m, const float* bias, float scale);
/* Measurement aid, no reference counterpart: a one-row run issues only its first `launches` launches (1: the gate/up
 * GEMV with the router; 2: and the down GEMV; 0 or 3: all three), so that a caller can time each launch inside the
 * layer's own sequence. Outputs of a shortened run are incomplete. */
int gfr_moe_set_launches(gfr_moe* m, int launches);
int gfr_moe_destroy(gfr_moe* m);

/* ---- The FP8 shared expert (moe.rs:132-167: shared_gu -> reduce8_bf16 -> shared_swiglu -> shared_down) -------
 * The reference's weights.layers[L].moe.shared.{gu,down}.{weight,scale} (front.rs:319-342 shapes; float8_e4m3fn,
 * OCP e4m3): gu [2 inter][hidden] (gate rows, then up rows), gu_scale [2 inter] bf16, down [hidden][inter],
 * down_scale [hidden] bf16; every pointer 16-byte aligned.
 * gfr_shared_fp8_run: input [rows][input_stride] bf16 -> out [rows][out_stride] fp32, in two launches:
 *   gu[r][n]  = bf16(sum over 8 contiguous K slices, in order, of gu_scale[n] * fp32 sum of input[r][k] * W[n][k])
 *               (the reference's fmm(shared_gu, sk = 8) + reduce8_bf16; its scalar oracle front.rs:190-217)
 *   act[r][i] = bf16(bf16(g / (1 + exp(-g))) * u), g = min(gu[r][i], 10), u = clamp(gu[r][inter + i], -10, 10)
 *               (shared_swiglu with limit 10; the formula of front.rs:669-675)
 *   out[r][n] = down_scale[n] * fp32 sum of act[r][k] * Wd[n][k]      (fmm(shared_down, sk = 1), fp32 output)
 * The sums inside a slice run in MFMA order, not the oracle's k order (within 1e-3 relative of it). hidden a multiple
 * of 512, inter of 64; input_stride a multiple of 8, out_stride of 4, both row pointers 16-byte aligned. The
 * reference's shared_swiglu also writes a `sums` buffer that nothing in the reference reads; it is not produced.
 * gfr_shared_fp8_gu / _act: the engine's last gu [max_rows][2 inter] and act [max_rows][inter] (bf16). */
typedef struct gfr_fp8_shared_weights {
    int hidden;
    int inter;
    const uint8_t* gu;
    const uint16_t* gu_scale;
    const uint8_t* down;
    const uint16_t* down_scale;
    const uint16_t* gu_bf16;     /* optional (NULL): the prefill form's bf16 copies, gfr_fp8_prepare_bf16 */
    const uint16_t* down_bf16;
} gfr_fp8_shared_weights;
/* The prefill form's weights (the reference's f8_b16_copy, prefill.cu:7-17, run by Gemms::prepare_f8,
 * prefill.rs:55-108): gu_bf16 [2 inter][hidden] and down_bf16 [hidden][inter] = bf16_rn(fp8(w) * row scale), written on
 * the stream; 16-byte aligned. Windows of more than 16 rows whose weights carry these copies run the reference's
 * prefill arithmetic (prefill.rs:127-150, batch.rs:1183-1195): gu = bf16(x . gu_bf16^T) and out = act . down_bf16^T as
 * library GEMMs (rocBLAS, fp32 accumulation) around the same SwiGLU; windows of up to 16 rows, or without the copies,
 * run the slice arithmetic above. The library may load a GEMM's code on the first call of a shape: make one eager
 * call of a window size before capturing it into a graph (the engine's workspace is set at create). */
int gfr_fp8_prepare_bf16(hipStream_t stream, const gfr_fp8_shared_weights* w, uint16_t* gu_bf16, uint16_t* down_bf16);
typedef struct gfr_shared_fp8 gfr_shared_fp8;
int gfr_shared_fp8_create(gfr_shared_fp8** out, int hidden, int inter, int max_rows);
int gfr_shared_fp8_run(gfr_shared_fp8* sh, hipStream_t stream, const gfr_fp8_shared_weights* w,
                       const uint16_t* input, int input_stride, int rows, float* out, int out_stride);
uint16_t* gfr_shared_fp8_gu(const gfr_shared_fp8* sh);
uint16_t* gfr_shared_fp8_act(const gfr_shared_fp8* sh);
int gfr_shared_fp8_destroy(gfr_shared_fp8* sh);
/* Moe::run_prefetched with its FP8 shared expert (moe.rs:66-182), for a layer made with gfr_moe_create_shared(...,
 * shared_exl3 = 0) and hidden a multiple of 512: the shared expert into the layer's own buffer
 * (gfr_moe_shared_output, [max_rows][hidden] fp32), then gfr_moe_run_shared with it. _router_fp8 computes the router
 * logits first, as gfr_moe_run_router. Input rows [rows][hidden] bf16, 16-byte aligned. */
int gfr_moe_run_fp8(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                    const float* logits, const gfr_fp8_shared_weights* sw, int rows);
int gfr_moe_run_router_fp8(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                           const uint16_t* router_weight, const gfr_fp8_shared_weights* sw, int rows);
float* gfr_moe_shared_output(const gfr_moe* m);

/* ---- The router alone (the reference's Triton topk, moe.rs:89-100; source absent, semantics of the benchmark):
 * logits [rows][routed] fp32 -> picks / weights [rows][topk + 1]: top-k by logit (ties: lower id), weights the
 * softmax over the k picks (summed in slot order), then the shared expert id `routed` with weight 1. */
/* GLM's gate, the arguments of the reference's `topk` call (moe.rs:89-99: logits, bias, picks, weights, 2.5), with
 * the published DeepSeek-V3 / GLM-4.5 "noaux" gating (its Triton source is not in the reference): score =
 * sigmoid(logit); top-k by score + bias[e] (ties: lower id); weight = score / (sum of the picked scores + 1e-20) *
 * scale, summed in slot order; shared expert last with weight 1. bias [routed] fp32. */
int gfr_route_topk_biased(hipStream_t stream, const float* logits, const float* bias, float scale, int rows,
                          int routed, int topk, int32_t* picks, float* weights);
int gfr_route_topk(hipStream_t stream, const float* logits, int rows, int routed, int topk, int32_t* picks,
                   float* weights);
/* Router logits (moe.rs:77-87, router_part [1,9,8] + router_sum; Triton, source absent): logits[r][e] =
 * sum over k of input[r][k] * router_weight[e][k], bf16 inputs, fp32 products and sums in a fixed order.
 * input [rows][input_stride] bf16, router_weight [routed][hidden] bf16, logits [rows][routed] fp32; hidden a
 * multiple of 8, at most 65536; input_stride a multiple of 8, input and router_weight 16-byte aligned (rows are read
 * 16 bytes at a time). */
int gfr_router_logits(hipStream_t stream, const uint16_t* input, int input_stride, const uint16_t* router_weight,
                      int hidden, int routed, int rows, float* logits);

/* ---- Single EXL3 linear (benchmark config 1; the decode path's GEMV with rot_in / down-epilogue formulas) ----
 * y [n] fp32 = svh * had(W^T xh) / sqrt(128), xh = fp16(had(x * suh) / sqrt(128)), x [kin] fp16. */
typedef struct gfr_linear gfr_linear;
int gfr_linear_create(gfr_linear** out, int kin, int n, int bits);
int gfr_linear_run(gfr_linear* l, hipStream_t stream, const uint16_t* x, const uint32_t* trellis,
                   const uint16_t* suh, const uint16_t* svh, float* y);
int gfr_linear_destroy(gfr_linear* l);

/* ---- The grouped trellis GEMV alone (exl3.cu:145-170 / :325-330, exl3_grouped_8_4) -------------------------
 * Z[((mat * SK + split) * P + pair) * N + n] = sum over split's k of X_mat[pair][k] * W_mat[uids[u]][k][n] for every
 * member pair of every distinct expert u < *ucount with uids[u] < experts; mats = 2 (X0/T0 gate, X1/T1 up) or 1.
 * X [P][kin] fp16 (rotated rows), trellis [experts][kin/16][n/16][8*bits]. SK = gfr_exl3_gemv_splits(kin) is fixed
 * by kin, so a row's result never depends on the other rows. maxu = grid bound on distinct experts; members are
 * read with stride maxm, 0 < maxm <= 64. */
int gfr_exl3_gemv_splits(int kin);
int gfr_exl3_grouped_gemv(hipStream_t stream, const uint16_t* x0, const uint16_t* x1, const uint32_t* t0,
                          const uint32_t* t1, const int32_t* uids, const int32_t* ucount, const int32_t* members,
                          float* z, int kin, int n, int pairs, int maxm, int slots, int experts, int bits, int mats,
                          int maxu);

/* ---- Debug / parity: the input rotation alone (rot_in, exl3.cu:224-241), bit-exact to the CPU restatement:
 * out[r][k] = fp16(had(x[r] * suh[expert[r]]) / sqrt(128)); x [rows][x_stride] bf16 (x_f16 = 0) or fp16;
 * suh [experts][k] fp16; k a multiple of 128. */
int gfr_exl3_rotate(hipStream_t stream, const uint16_t* x, int x_stride, int x_f16, const int32_t* expert,
                    const uint16_t* suh, int k, int rows, uint16_t* out);

/* ---- Debug / parity: decoded fp16 weights of one matrix [kin][n] (row = k), bit-exact to experts.rs:47-74 ---- */
int gfr_exl3_decode_tiles(hipStream_t stream, const uint32_t* trellis, int kin, int n, int bits, uint16_t* out);

/* ---- Cache-warming reads of weight memory (native/l2-prefetch/bridge.cpp:11-45, l2pf.cu) ----------------------
 * Read hints only: the kernels load one dword of every 128-byte line of the given ranges and write nothing, so no
 * result can change. On MI355X a line read lands in the reading XCD's L2 and in the 256 MB memory-side cache, from
 * which the expert launches on every XCD then read it. Meant for a side stream forked from the caller's main stream
 * right after grouped routing (the reference's l2_prefetch.rs Owner::experts), joined before the routed experts'
 * results are needed; nothing here synchronises or allocates, so the launches can be captured into a graph.
 * Preconditions return GFR_EINVAL where the reference returns cudaErrorInvalidValue. */
#define GFR_PREFETCH_EXPERT_BYTES_MAX 65536
uint32_t gfr_prefetch_abi(void);                                     /* alaska_l2pf_abi, bridge.cpp:11: 1 */
/* alaska_l2pf_properties, bridge.cpp:12-20: the current device's CU count and L2 size in bytes (one XCD's L2). */
int gfr_prefetch_properties(int* cus, int* l2_bytes);
/* alaska_l2pf_capturing, bridge.cpp:21-29: *active = 1 while the stream is being captured; an invalidated capture
 * returns hipErrorStreamCaptureInvalidated. */
int gfr_prefetch_capturing(hipStream_t stream, int* active);
/* alaska_l2pf_segments, bridge.cpp:30-35: table = device array of count (address, bytes) int64 pairs, each
 * 16-byte aligned with bytes a positive multiple of 16 (entries that are not are skipped); grid workgroups of 128
 * threads. The 128-byte lines of all segments are numbered in table order and dealt to the grid's threads: thread t
 * reads lines t, t + threads, t + 2 threads, ... */
int gfr_prefetch_segments(const int64_t* table, int count, int grid, hipStream_t stream);
/* alaska_l2pf_experts, bridge.cpp:36-45: for u < min(*count, maxu) (device values), the first `bytes` of expert
 * ids[u] in the gate and up trellis tensors bases[0] and bases[1] (device array of 2 addresses), at
 * bases[m] + ids[u] * stride; ids outside [0, experts) are skipped. bytes in (0, min(stride,
 * GFR_PREFETCH_EXPERT_BYTES_MAX)], bytes and stride multiples of 16, grid > 0. */
int gfr_prefetch_experts(const int32_t* ids, const int32_t* count, int maxu, const int64_t* bases, int64_t stride,
                         int64_t bytes, int64_t experts, int grid, hipStream_t stream);

/* ---- Prepared weights (src/prepared.rs) ------------------------------------------------------------------------
 * The reference's prepared format: a JSON manifest {format: 1, file_size, chunk, chunk_sha256[], storages[], tree,
 * key} next to data.bin (prepared.rs:15-40). Tensor paths are the reference's ("weights.layers[3].moe.experts.gt").
 * open     = Prepared::open_parts + the tree walk (prepared.rs:101-132, 186-230): storages ascending, non-overlapping,
 *            inside data.bin; every tensor view inside its storage and on its storage's device. The reference's
 *            model-identity checks (model name, TP4 rank, GLM geometry, :151-185) are not applied: they belong to its
 *            full model.
 * load     = Prepared::load_selected (:270-366): storages holding a tensor under one of the prefixes (all when
 *            nprefixes = 0), data.bin read in manifest-chunk pieces through pinned staging, each needed piece checked
 *            against its SHA-256 before it is copied; keeps 8 GiB of device memory free. Allocates (hipMalloc).
 * pointer  = Loaded::pointer (:369-377); expect = Prepared::expect (:236-248); read_tensor = read_tensor_segment
 *            (:253-266, from disk, no device needed); experts = the weights.layers[L].moe.experts.* lookups of
 *            ExpertGpu::run_rows (experts.rs:467) with the shapes of experts::probe (:146-156), any E / hidden / inter /
 *            bits. Not thread-safe; one prepared model per thread. */
#define GFR_TENSOR_MAX_RANK 8
typedef struct gfr_tensor_info {
    int storage;
    char dtype[24];
    int rank;
    uint64_t shape[GFR_TENSOR_MAX_RANK];
    uint64_t stride[GFR_TENSOR_MAX_RANK];
    uint64_t off;            /* element offset into the storage */
    int cuda;                /* 1: device storage, 0: host ("cpu") */
    uint64_t extent_bytes;   /* Tensor::extent (prepared.rs:51-71) */
} gfr_tensor_info;
typedef struct gfr_prepared gfr_prepared;
int gfr_prepared_open(gfr_prepared** out, const char* manifest_path);
int gfr_prepared_tensor_count(const gfr_prepared* p);
const char* gfr_prepared_tensor_name(const gfr_prepared* p, int i);           /* path order */
int gfr_prepared_tensor(const gfr_prepared* p, const char* path, gfr_tensor_info* info);
int gfr_prepared_expect(const gfr_prepared* p, const char* path, const char* dtype, const uint64_t* shape, int rank);
int gfr_prepared_read_tensor(const gfr_prepared* p, const char* path, uint64_t offset, uint64_t len, void* host_out);
int gfr_prepared_load(gfr_prepared* p, const char* const* prefixes, int nprefixes);
int gfr_prepared_loaded(const gfr_prepared* p, uint64_t* device_bytes, double* seconds);
int gfr_prepared_pointer(const gfr_prepared* p, const char* path, void** device_ptr);
int gfr_prepared_experts(const gfr_prepared* p, int layer, gfr_exl3_experts* out);
/* The weights.layers[L].moe.shared.{gu,down}.{weight,scale} lookups of moe.rs:136-161 (float8_e4m3fn weights, bf16
 * scales, any hidden / inter); GFR_EINVAL when a tensor is missing or has another dtype or shape. */
int gfr_prepared_shared_fp8(const gfr_prepared* p, int layer, gfr_fp8_shared_weights* out);
int gfr_prepared_destroy(gfr_prepared* p);
/* The format's hash: lowercase hex SHA-256 (FIPS 180-4) of a host buffer into out65 (64 digits + NUL). */
int gfr_sha256_hex(const void* data, uint64_t len, char* out65);
/* Tensor::extent (prepared.rs:51-71) of a described view: bytes from the storage start past its last element;
 * GFR_EINVAL on a rank mismatch, an unknown dtype or overflow. */
int gfr_tensor_extent(const char* dtype, const uint64_t* shape, const uint64_t* stride, int shape_rank,
                      int stride_rank, uint64_t off, uint64_t* bytes);

#ifdef __cplusplus
}
#endif
#endif
