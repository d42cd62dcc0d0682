// Router of the benchmark configs, one wave a token (the reference runs a precompiled Triton `topk`, glm-flash-rs
// src/moe.rs:89-100, whose source is absent): top-k of the routed logits by value (ties: the lower id), weights =
// softmax over the k picks (exp(l - l_max) / sum, summed in slot order), then the shared expert with weight 1.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "exl3_format.hpp"

namespace gfr {

constexpr int ROUTE_MAX_E = 64 * 16;

// One wave (64 lanes) routes one token into registers: lane s < topk holds the s-th pick and its weight, lane topk
// the shared expert (weight 1). k rounds of a wave-wide max (DPP / permlane, no LDS), ties to the lower id.
__device__ __forceinline__ void route_token_regs(const float* __restrict__ l, int E, int topk, int shared_id,
                                                 int& pick, float& weight) {
    constexpr int PER = ROUTE_MAX_E / 64;
    const int lane = threadIdx.x & 63;
    const int per = (E + 63) >> 6;                     // values a lane actually holds
    float v[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = j * 64 + lane;
        v[j] = (j < per && e < E) ? l[e] : -__builtin_inff();
    }
    float my_v = 0.f;                                  // lane s < topk: the s-th pick's logit and id
    int my_e = 0;
    for (int s = 0; s < topk; ++s) {
        float lm = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < PER; ++j)
            if (j < per) lm = fmaxf(lm, v[j]);
        const float best = wave_max(lm);
        int le = 0x7fffffff;                           // this lane's lowest id holding the best value
#pragma unroll
        for (int j = PER - 1; j >= 0; --j)
            if (j < per && v[j] == best && j * 64 + lane < E) le = j * 64 + lane;
        const int be = wave_min(le);
        if ((be & 63) == lane) {
#pragma unroll
            for (int j = 0; j < PER; ++j)
                if (j == (be >> 6)) v[j] = -__builtin_inff();
        }
        if (lane == s) {
            my_v = best;
            my_e = be;
        }
    }
    const float top = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_v), 0));
    const float ex = lane < topk ? expf(my_v - top) : 0.f;
    float sum = 0.f;
    for (int s = 0; s < topk; ++s) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), s));
    pick = lane < topk ? my_e : shared_id;
    weight = lane < topk ? ex / sum : 1.f;
}

// One wave routes one token; pk / wt (LDS or global) receive topk + 1 entries.
__device__ __forceinline__ void route_token(const float* __restrict__ l, int E, int topk, int shared_id, int* pk,
                                            float* wt) {
    int pick;
    float weight;
    route_token_regs(l, E, topk, shared_id, pick, weight);
    const int lane = threadIdx.x & 63;
    if (lane <= topk) {
        pk[lane] = pick;
        wt[lane] = weight;
    }
}

}  // namespace gfr
