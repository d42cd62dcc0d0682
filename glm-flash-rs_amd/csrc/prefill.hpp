// Prefill-chunk experts (FastExperts, glm-flash-rs src/fast_experts.rs:27-208) on gfx950: engine interface used by
// the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/gfr_moe.h"

namespace gfr {

struct PrefillDims {
    int hidden, inter, slots, exl3_slots, experts, max_rows;
};

hipError_t prefill_create(gfr_fast_experts** out, int hidden, int inter, int slots, int exl3_slots, int experts,
                          int max_rows);
PrefillDims prefill_dims(const gfr_fast_experts* fx);
hipError_t prefill_run(gfr_fast_experts* fx, hipStream_t s, const gfr_exl3_experts* w, const uint16_t* input,
                       int input_stride, const int* picks, const int* ids, const int* count, const int* members,
                       int rows, int maxm, bool shared_x, const float* combine_weights = nullptr,
                       float* combine_out = nullptr, bool* combined = nullptr, bool planned = false,
                       const float* combine_shared = nullptr, int shared_stride = 0,
                       hipEvent_t shared_ready = nullptr,    // the stream waits on it before the combine
                       bool rotated = false);                // the rows are already rotated (launch_route_group_rot)
// The large-window grouping (launch_group_large with its item plan) with prefill_run's input rotation in its last
// launch, for a window of the Moe path whose picks are routed; prefill_run then runs with planned and rotated.
// Returns hipErrorNotSupported where the window does not fit (the caller then launches the parts).
hipError_t launch_group_large_rot(gfr_fast_experts* fx, hipStream_t s, const gfr_exl3_experts* w,
                                  const uint16_t* input, int input_stride, const int* picks, int rows, int slots,
                                  int E, uint32_t* bits, uint8_t* first, int* prefix, int* counts, int* ids,
                                  int* count, int* members, int maxm);
// Route + group + item plan (launch_route_group's work) and prefill_run's input rotation in one launch, for a
// window of the Moe path (the two input rotations apart); prefill_run then runs with planned and rotated. Returns
// hipErrorNotSupported where the window does not fit the fused form (the caller then launches the parts).
hipError_t launch_route_group_rot(gfr_fast_experts* fx, hipStream_t s, const gfr_exl3_experts* w,
                                  const uint16_t* input, int input_stride, const float* logits, int rows, int routed,
                                  int topk, int* picks, float* weights, int* ids, int* count, int* members, int maxm,
                                  const float* bias, float scale);
// The item plan of a window of `rows` at `bits`: member rows an item, and the buffers prefill_run's GEMMs read
// (ucnt, items, plan). A caller that fills them itself (the fused route + group launch) passes planned = true.
int prefill_item_rows(const gfr_fast_experts* fx, int rows, int bits);
void prefill_plan_buffers(gfr_fast_experts* fx, int** ucnt, int** items, int** plan);
float* prefill_output(const gfr_fast_experts* fx);
uint16_t* prefill_xd(const gfr_fast_experts* fx);
uint16_t* prefill_rotated(const gfr_fast_experts* fx, int mat);
void prefill_destroy(gfr_fast_experts* fx);

}  // namespace gfr
