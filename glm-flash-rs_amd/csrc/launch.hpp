// Host-side launchers of the gfx950 kernels (one per kernel family); the C ABI in gfr_moe_api.hip calls these.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gfr {

// grouping.hip
constexpr int GROUP_SMALL_ROWS = 256;
constexpr size_t GROUP_LDS_MAX = 65536;   // dynamic LDS a grouping launch may ask for
size_t group_small_lds(int rows, int slots, int E);   // LDS of launch_group_small
size_t route_group_lds(int rows, int slots, int E);   // LDS of launch_route_group
hipError_t launch_group_small(hipStream_t s, const int* picks, int rows, int slots, int E, int* ids, int* count,
                              int* members, int maxm);
// route (route.hpp) + group_small in one launch; rows <= GROUP_SMALL_ROWS, routed + 1 <= 1024
// with plan != nullptr it also writes the prefill engine's item plan for bm-row items (prefill_plan_buffers) over
// the experts below plan_E (those the weights hold)
hipError_t launch_route_group(hipStream_t s, const float* logits, int rows, int routed, int topk, int* picks,
                              float* weights, int* ids, int* count, int* members, int maxm, int bm = 0,
                              int* plan_ucnt = nullptr, int* plan_items = nullptr, int* plan = nullptr,
                              int plan_E = 0, const float* bias = nullptr, float scale = 1.f);
// With plan (bm rows an item) the scatter launch also writes the prefill engine's item plan over the experts below
// plan_E (those the weights hold).
hipError_t launch_group_large(hipStream_t s, const int* picks, int rows, int slots, int E, uint32_t* bits,
                              uint8_t* first, int* prefix, int* counts, int* ids, int* count, int* members, int maxm,
                              int bm = 0, int* plan_ucnt = nullptr, int* plan_items = nullptr, int* plan = nullptr,
                              int plan_E = 0, bool scatter = true);
// scatter = false: the mark and prefix launches only (the caller launches the scatter, group_scatter_body, itself)

// exl3_decode.hip
hipError_t launch_decode_tiles(hipStream_t s, const uint32_t* T, int kin, int n, int bits, uint16_t* out);
// in_f16: x is fp16 (the single-linear config) instead of bf16 (the reference's rot_in)
hipError_t launch_rot_in(hipStream_t s, const uint16_t* x, int x_stride, bool in_f16, const int* pick,
                         const uint16_t* suh0, const uint16_t* suh1, uint16_t* out0, uint16_t* out1, int K, int P,
                         int slots, int exl3_slots, int mats);
int gemv_splits(int Kin);  // K splits of the decode GEMV (fixed by the shape, so a row's bits never depend on rows)
hipError_t launch_gemv(hipStream_t s, const uint16_t* X0, const uint16_t* X1, const uint32_t* T0, const uint32_t* T1,
                       const int* uids, const int* ucount, const int* members, float* Z, int Kin, int N, int P,
                       int maxm, int slots, int E, int bits, int mats, int maxu);
int gemv_gateup_splits(int D);  // K splits of the decode gate/up GEMV (one 128-block a wave, 4 waves)
int gemv_down_splits(int N);    // k-block parts of the decode down GEMV (one a 128-k block)
// Decode path: gate/up GEMV with rot_in fused (-> gate/up split partials Zgu [2][SK][P][N]); down GEMV with the
// gate/up epilogue fused as its activation source and the down epilogue's transform applied to each k-block part
// (-> Zd [N / 128][P][D], xd [P][N]); the parts' sum + combine.
// One-token windows can route inside the gate/up launch: the token's logits, and where to store its picks /
// weights and the window's grouping (ids, count, members with stride maxm) for the later launches.
struct RouteOne {
    const float* logits;
    const float* bias;        // the gate (route.hpp RouteGate): nullptr = softmax
    float scale;
    int routed;
    int* picks;
    float* weights;
    int* ids;
    int* count;
    int* members;
};
// The layer's FP8 shared expert when it rides on a one-token window's launches (shared_fp8.hpp): the shared slot's
// workgroups of the gate/up launch write gu / act, those of the down launch out [hidden] (fp32).
struct Fp8Shared {
    const uint8_t* gu_w;
    const uint16_t* gu_s;
    const uint8_t* d_w;
    const uint16_t* d_s;
    uint16_t* gu;
    uint16_t* act;
    float* out;
    int hidden, inter;
};
hipError_t launch_expert_gateup(hipStream_t s, const uint16_t* x, int x_stride, const uint16_t* suh_g,
                                const uint16_t* suh_u, const uint32_t* gt, const uint32_t* ut, const int* uids,
                                const int* ucount, const int* members, float* Zgu, int D, int N, int P, int rows,
                                int maxm, int slots, int E, int bits, int maxu, const RouteOne* route,
                                const uint32_t* dt_next = nullptr, const Fp8Shared* fp8 = nullptr);
// dt_next: the layer's down trellis; the gate waves read each window expert's down matrix once into the caches
// after their own work (expert_gemv_kernel), so the down launch's first loads hit the memory-side cache
// SKgu: the gate/up partials' K splits (gemv_gateup_splits)
hipError_t launch_expert_down(hipStream_t s, const float* Zgu, int D, int SKgu, const uint16_t* svh_g,
                              const uint16_t* svh_u, const uint16_t* suh_d, float limit, uint16_t* xd,
                              const uint32_t* dt, const uint16_t* svh_d, const int* uids, const int* ucount,
                              const int* members, float* Zd, int N, int P, int rows, int maxm, int slots, int E,
                              int bits, int maxu, const RouteOne* route = nullptr, const Fp8Shared* fp8 = nullptr);
// route: the one-token window was routed by the gate/up launch (its picks); the down launch then runs one program a
// slot and reads no grouping table
// Finish of the decode path: Zd's transformed k-block parts [N / 128][P][D] added in order -> y; with weights the
// slot-ordered combine -> out
hipError_t launch_sum_finish(hipStream_t s, const float* Zd, float* y, int rows, int P, int D, int SK, int slots,
                             int exl3_slots, const float* weights, const float* shared, int shared_stride,
                             float* out);
// one fp16 row through one linear with the input rotation fused (partials for down_epilogue)
int gemv_linear_splits(int kin);
hipError_t launch_linear_fused(hipStream_t s, const uint16_t* x, const uint16_t* suh, const uint32_t* trellis,
                               const int* uids, const int* ucount, const int* members, float* z, int kin, int n,
                               int bits);
hipError_t launch_down_finish(hipStream_t s, const float* Zd, const int* pick, const uint16_t* svh_d, float* y,
                              int rows, int P, int D, int SK, int slots, int exl3_slots, const float* weights,
                              const float* shared, int shared_stride, float* out);
// pair_order: xd in the MFMA path's pair order (x[m + 8], x[m] within each 16-value tile) instead of k order
hipError_t launch_gateup_epilogue(hipStream_t s, const float* Z, const int* pick, const uint16_t* svh_g,
                                  const uint16_t* svh_u, const uint16_t* suh_d, uint16_t* xd, int P, int N, int SK,
                                  int slots, int exl3_slots, float limit, bool pair_order = false);
hipError_t launch_down_epilogue(hipStream_t s, const float* Z, const int* pick, const uint16_t* svh_d, float* y,
                                int P, int D, int SK, int slots, int exl3_slots);


// router.hip
// bias == nullptr: the softmax gate; else GLM's sigmoid + bias gate with weights times scale (route.hpp RouteGate)
hipError_t launch_route(hipStream_t s, const float* logits, int rows, int E, int topk, int shared_id, int* picks,
                        float* weights, const float* bias = nullptr, float scale = 1.f);
// shared: the caller's output for the slots s >= exl3_slots ([rows][shared_stride] fp32), or null
hipError_t launch_combine(hipStream_t s, const float* y, const float* weights, int rows, int slots, int exl3_slots,
                          int D, const float* shared, int shared_stride, float* out);
// logits [rows][E] fp32 = x [rows][x_stride] bf16 times W [E][D] bf16 (D a multiple of 8, at most
// router_logits_max_hidden())
int router_logits_max_hidden();
hipError_t launch_router_logits(hipStream_t s, const uint16_t* x, int x_stride, const uint16_t* W, int D, int E,
                                int rows, float* logits);

// shared_fp8.hip
// The reference's FP8 shared expert (moe.rs:132-167) for rows [rows][x_stride] bf16: gate/up (8 K slices, bf16 gu
// [rows][2 inter], limited SwiGLU -> act [rows][inter] bf16), then down -> out [rows][out_stride] fp32. hidden a
// multiple of 512, inter of 64; x, out, the weights and the scales 16-byte aligned, x_stride % 8 == 0,
// out_stride % 4 == 0.
hipError_t launch_shared_fp8(hipStream_t s, const uint8_t* wgu, const uint16_t* sgu, const uint8_t* wd,
                             const uint16_t* sd, const uint16_t* x, int x_stride, int rows, int hidden, int inter,
                             uint16_t* gu, uint16_t* act, float* out, int out_stride);
// The prefill form: the reference's bf16 weight copies (f8_b16_copy, prefill.cu:7-17: bf16(fp8 * row scale)), and
// the expert as two library GEMMs on them around shared_swiglu (blas: a rocblas_handle with its workspace set).
hipError_t launch_fp8_b16_copy(hipStream_t s, const uint8_t* w, const uint16_t* scale, uint16_t* out, int n, int k);
hipError_t launch_shared_fp8_prefill(void* blas, hipStream_t s, const uint16_t* wgu16, const uint16_t* wd16,
                                     const uint16_t* x, int x_stride, int rows, int hidden, int inter, uint16_t* gu,
                                     uint16_t* act, float* out, int out_stride);

}  // namespace gfr
