// Router of the benchmark configs, one wave a token (the reference runs a precompiled Triton `topk`, glm-flash-rs
// src/moe.rs:89-100, whose source is absent): top-k of the routed logits by value (ties: the lower id), weights =
// softmax over the k picks (exp(l - l_max) / sum, summed in slot order), then the shared expert with weight 1.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "exl3_format.hpp"

namespace gfr {

constexpr int ROUTE_MAX_E = 64 * 16;

// The router's gate. bias == nullptr: the benchmark's softmax gate (top-k by logit, softmax over the picks).
// Otherwise GLM's gate, the arguments of the reference's `topk` call (moe.rs:89-99: logits, bias, picks, weights,
// 2.5), with the published DeepSeek-V3 / GLM-4.5 "noaux" gating: scores = sigmoid(logit); selection by
// score + bias[e]; weights = score / (sum of the k picked scores + 1e-20) * scale.
struct RouteGate {
    const float* bias;
    float scale;
};
__device__ __forceinline__ float sigmoidf_(float x) { return 1.f / (1.f + expf(-x)); }

// The router's inputs of one token in registers: lane l holds logits l, l + 64, ... (PER of them), and with GLM's gate
// the matching biases. Loading them is split from the selection so that a caller can issue other loads in between.
template <int PER>
struct RouteIn {
    float l[PER];
    float b[PER];
};
// Every load is issued by every lane (clamped index, the logits standing in for a missing bias), so that the number of
// loads in flight is the same on every path and a caller's later waits need not be conservative.
template <int PER>
__device__ __forceinline__ void route_load(const float* __restrict__ l, int E, RouteGate g, RouteIn<PER>& in) {
    const int lane = threadIdx.x & 63;
    const float* bias = g.bias ? g.bias : l;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = j * 64 + lane < E ? j * 64 + lane : E - 1;
        in.l[j] = l[e];
        in.b[j] = bias[e];
    }
}

// One wave (64 lanes) routes one token into registers: lane s < topk holds the s-th pick and its weight, lane topk
// the shared expert (weight 1). k rounds of a wave-wide max (DPP / permlane, no LDS) whose winner is the lowest id
// holding it: from 65 to 256 experts over each lane's sorted scores, otherwise a ballot per register (at 64 and
// fewer the ballot is the cheaper of the two: 19.00 against 18.95 us a config-2 layer).
// need_weight == false (uniform over the wave): the picks only, weight left 0 (callers that only need the experts).
template <int PER>
__device__ __forceinline__ void route_pick(const RouteIn<PER>& in, const float* __restrict__ l, int E, int topk,
                                           int shared_id, int& pick, float& weight, RouteGate g,
                                           bool need_weight = true) {
    const int lane = threadIdx.x & 63;
    float v[PER];
    // a uniform branch: the softmax gate skips the sigmoids (selected after the fact, they were computed anyway)
    if (g.bias) {
#pragma unroll
        for (int j = 0; j < PER; ++j)
            v[j] = j * 64 + lane < E ? sigmoidf_(in.l[j]) + in.b[j] : -__builtin_inff();
    } else {
#pragma unroll
        for (int j = 0; j < PER; ++j) v[j] = j * 64 + lane < E ? in.l[j] : -__builtin_inff();
    }
    float my_v = 0.f;                                  // lane s < topk: the s-th pick's logit and id
    int my_e = 0;
    if constexpr (PER == 2 || PER == 4) {
        // Each lane's PER scores sorted once, highest first (equal scores: lower id first). A round then takes the
        // wave-wide maximum of the lanes' heads; its lane pops its head. Equal maxima on several lanes (rare) go to
        // the lowest id among them. The same picks as the scan below, in fewer operations a round.
        int id[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) id[j] = j * 64 + lane;
        auto cx = [&](int a_, int b_) {
            const bool sw = v[b_] > v[a_] || (v[b_] == v[a_] && id[b_] < id[a_]);
            const float tv = v[a_];
            const int ti = id[a_];
            v[a_] = sw ? v[b_] : v[a_];
            id[a_] = sw ? id[b_] : id[a_];
            v[b_] = sw ? tv : v[b_];
            id[b_] = sw ? ti : id[b_];
        };
        if constexpr (PER == 2) cx(0, 1);
        if constexpr (PER == 4) {
            cx(0, 1); cx(2, 3); cx(0, 2); cx(1, 3); cx(1, 2);
        }
        for (int s = 0; s < topk; ++s) {
            const float best = wave_max_nn(v[0]);     // scores are finite or -inf
            const uint64_t c = __ballot(v[0] == best);
            int w = __builtin_ctzll(c);
            if (__popcll(c) > 1) {
                int m = v[0] == best ? id[0] : 0x7fffffff;
                m = min(m, (int)lane_xor<1>((uint32_t)m));
                m = min(m, (int)lane_xor<2>((uint32_t)m));
                m = min(m, (int)lane_xor<4>((uint32_t)m));
                m = min(m, (int)lane_xor<8>((uint32_t)m));
                m = min(m, (int)lane_xor<16>((uint32_t)m));
                m = min(m, (int)lane_xor<32>((uint32_t)m));
                w = __builtin_ctzll(__ballot(v[0] == best && id[0] == m));
            }
            const int be = __builtin_amdgcn_readlane(id[0], w);
            if (lane == w) {
#pragma unroll
                for (int j = 0; j + 1 < PER; ++j) {
                    v[j] = v[j + 1];
                    id[j] = id[j + 1];
                }
                v[PER - 1] = -__builtin_inff();
            }
            if (lane == s) {
                my_v = best;
                my_e = be;
            }
        }
    } else {
        for (int s = 0; s < topk; ++s) {
            float lm = v[0];
#pragma unroll
            for (int j = 1; j < PER; ++j) lm = max_nn(lm, v[j]);
            const float best = wave_max_nn(lm);       // scores are finite or -inf
            int be = 0;
#pragma unroll
            for (int j = PER - 1; j >= 0; --j) {       // the lowest register (id block) holding it wins
                const uint64_t b = __ballot(v[j] == best && j * 64 + lane < E);
                if (b) be = j * 64 + __builtin_ctzll(b);
            }
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
    }
    pick = lane < topk ? my_e : shared_id;
    weight = 0.f;
    if (!need_weight) return;
    if (g.bias) {
        // the picked experts' unbiased scores, normalised over the picks in slot order, times the scale
        const float sc = lane < topk ? sigmoidf_(l[my_e]) : 0.f;
        float sum = 0.f;
        for (int s = 0; s < topk; ++s) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, sc), s));
        weight = lane < topk ? sc / (sum + 1e-20f) * g.scale : 1.f;
        return;
    }
    const float top = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_v), 0));
    const float ex = lane < topk ? expf(my_v - top) : 0.f;
    float sum = 0.f;
    for (int s = 0; s < topk; ++s) sum += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), s));
    weight = lane < topk ? ex / sum : 1.f;
}

template <int PER>
__device__ __forceinline__ void route_token_per(const float* __restrict__ l, int E, int topk, int shared_id,
                                                int& pick, float& weight, RouteGate g, bool need_weight) {
    RouteIn<PER> in;
    route_load<PER>(l, E, g, in);
    route_pick<PER>(in, l, E, topk, shared_id, pick, weight, g, need_weight);
}

__device__ __forceinline__ void route_token_regs(const float* __restrict__ l, int E, int topk, int shared_id,
                                                 int& pick, float& weight, RouteGate g = {nullptr, 1.f},
                                                 bool need_weight = true) {
    if (E <= 64) route_token_per<1>(l, E, topk, shared_id, pick, weight, g, need_weight);
    else if (E <= 128) route_token_per<2>(l, E, topk, shared_id, pick, weight, g, need_weight);
    else if (E <= 256) route_token_per<4>(l, E, topk, shared_id, pick, weight, g, need_weight);
    // above 256: as many registers a lane as the experts need (each round scans every register, and GLM's gate takes
    // a sigmoid of each: 288 experts in 5 instead of 16)
    else if (E <= 320) route_token_per<5>(l, E, topk, shared_id, pick, weight, g, need_weight);
    else if (E <= 512) route_token_per<8>(l, E, topk, shared_id, pick, weight, g, need_weight);
    else route_token_per<ROUTE_MAX_E / 64>(l, E, topk, shared_id, pick, weight, g, need_weight);
}

// One wave routes one token; pk / wt (LDS or global) receive topk + 1 entries.
__device__ __forceinline__ void route_token(const float* __restrict__ l, int E, int topk, int shared_id, int* pk,
                                            float* wt, RouteGate g = {nullptr, 1.f}) {
    int pick;
    float weight;
    route_token_regs(l, E, topk, shared_id, pick, weight, g);
    const int lane = threadIdx.x & 63;
    if (lane <= topk) {
        pk[lane] = pick;
        wt[lane] = weight;
    }
}

}  // namespace gfr
