// Device bodies of the grouping launches, shared by the grouping kernels (grouping.hip) and the prefill engine's
// launches that also rotate the input (exl3_prefill.hip): one-workgroup routing and grouping of small windows
// (rows <= GROUP_SMALL_ROWS) and the per-expert scatter of large ones. The grouping is bit-exact to glm-flash-rs
// native/grouping.cu and to src/grouping.rs:141-192 (contract in grouping.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "route.hpp"

namespace gfr {

// Inclusive scan of x over the wave: DPP row shifts by 1, 2, 4, 8 inside each 16-lane row (lanes past the row's
// start read 0), then the gfx9 row broadcasts (lane 15 of rows 0 and 2 into rows 1 and 3, lane 31 into rows 2 and 3).
__device__ __forceinline__ int wave_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return x;
}

// Inclusive scan of x over the workgroup (blockDim.x a multiple of 64, at most 1024). `scratch` holds 16 ints,
// 16-byte aligned. Returns the inclusive prefix; *total receives the sum. The wave totals are read back as four
// 16-byte LDS loads issued together.
__device__ __forceinline__ int block_scan(int x, int* scratch, int* total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    x = wave_scan(x);
    if (lane == 63) scratch[wave] = x;
    __syncthreads();
    int4 q[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = reinterpret_cast<const int4*>(scratch)[j];
    const int t[16] = {q[0].x, q[0].y, q[0].z, q[0].w, q[1].x, q[1].y, q[1].z, q[1].w,
                       q[2].x, q[2].y, q[2].z, q[2].w, q[3].x, q[3].y, q[3].z, q[3].w};
    int off = 0, all = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const int v = w < nw ? t[w] : 0;
        off += w < wave ? v : 0;
        all += v;
    }
    __syncthreads();
    *total = all;
    return x + off;
}

// One workgroup (blockDim.x a multiple of 64, <= 1024). lds: E * ceil(rows / 32) bitmap words + 2 E ints.
// picks may live in LDS or global memory.
// With `plan` (the prefill engine's item plan, bm rows an item): plan_ucnt[u] = members of used expert u,
// plan_items[k] = (u << 16) | pass over the ceil(count / bm) passes of each u in u order, plan[0] = item count -- what
// prefill_plan_kernel derives from the members table, here from the counts already in LDS.
__device__ __forceinline__ void group_small_body(const int* picks, int rows, int slots, int E, int* __restrict__ ids,
                                                 int* __restrict__ count, int* __restrict__ members, int maxm,
                                                 uint32_t* lds, int* scan_scratch, int bm = 0,
                                                 int* __restrict__ plan_ucnt = nullptr,
                                                 int* __restrict__ plan_items = nullptr, int* __restrict__ plan = nullptr,
                                                 int plan_E = 0) {
    const int NWD = (rows + 31) >> 5;
    uint32_t* bits = lds;                                    // [E][NWD]
    int* ucnt = reinterpret_cast<int*>(lds + (size_t)E * NWD);  // [E]: count of the u-th used expert
    int* place = ucnt + E;                                   // [E]: u of expert e, or -1
    for (int i = threadIdx.x; i < E * NWD; i += blockDim.x) bits[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < rows * slots; i += blockDim.x) {
        const int r = i / slots, e = picks[i];
        if (e >= 0 && e < E) atomicOr(&bits[e * NWD + (r >> 5)], 1u << (r & 31));
    }
    __syncthreads();
    // experts in rounds of blockDim.x: count, then the ascending order of the used ones
    int base = 0, base_w = 0;
    for (int e0 = 0; e0 < E; e0 += blockDim.x) {
        const int e = e0 + threadIdx.x;
        int c = 0;
        if (e < E)
            for (int w = 0; w < NWD; ++w) c += __popc(bits[e * NWD + w]);
        // one scan of both counts: used experts (low 16 bits) and, for the plan, the used experts the weights hold
        // (ids below plan_E, high 16 bits); a round has at most 1024 experts, so neither field carries over
        int packed_total;
        const int packed = block_scan((c > 0 ? 1 : 0) | (plan && c > 0 && e < plan_E ? 1 << 16 : 0), scan_scratch,
                                      &packed_total);
        const int incl = packed & 0xffff, total = packed_total & 0xffff;
        base_w += packed_total >> 16;
        if (e < E) {
            place[e] = c > 0 ? base + incl - 1 : -1;
            if (c > 0) {
                ids[base + incl - 1] = e;
                ucnt[base + incl - 1] = c;
            }
        }
        base += total;
    }
    __syncthreads();
    const int used = base;
    if (threadIdx.x == 0) *count = used;
    if (plan) {
        int ibase = 0;
        for (int u0 = 0; u0 < used; u0 += blockDim.x) {
            const int u = u0 + threadIdx.x;
            // ids ascend, so the experts the weights hold are the first base_w; the others (a shared expert that is
            // not EXL3) get no items, as in prefill_plan_kernel
            const int c = u < used ? ucnt[u] : 0, np = u < base_w ? (c + bm - 1) / bm : 0;
            int total;
            const int first = ibase + block_scan(np, scan_scratch, &total) - np;
            if (u < used) {
                plan_ucnt[u] = c;
                for (int k = 0; k < np; ++k) plan_items[first + k] = (u << 16) | k;
            }
            ibase += total;
        }
        if (threadIdx.x == 0) plan[0] = ibase;
    }
    // members: thread per (row, slot); the first slot of row r holding expert e writes code r * 32 + slot at the
    // row's rank among e's rows (the popcount of e's bitmap below bit r) -- no serial walk over an expert's rows
    for (int i = threadIdx.x; i < rows * slots; i += blockDim.x) {
        const int r = i / slots, sl = i - r * slots, e = picks[i];
        if (e < 0 || e >= E) continue;
        bool first = true;
        for (int q = 0; q < sl; ++q) first &= picks[r * slots + q] != e;
        if (!first) continue;
        const uint32_t* be = bits + e * NWD;
        int off = __popc(be[r >> 5] & ((1u << (r & 31)) - 1u));
        for (int q = 0; q < (r >> 5); ++q) off += __popc(be[q]);
        members[(size_t)place[e] * maxm + off] = r * 32 + sl;
    }
    // every other entry of the E x maxm table is -1
    const int total = E * maxm;
    for (int i = threadIdx.x; i < total; i += blockDim.x) {
        const int u = i / maxm, j = i - u * maxm;
        if (u >= used || j >= ucnt[u]) members[i] = -1;
    }
}


// The workgroup's waves route rows r = wave, wave + waves, ... into pk / wt (topk + 1 entries a row); a wave's next
// row's logits are loaded before it routes the current one, so the loads of consecutive rows overlap.
template <int PER>
__device__ __forceinline__ void route_rows(const float* __restrict__ logits, int rows, int routed, int topk, int* pk,
                                           float* wt, RouteGate gate) {
    const int lane = threadIdx.x & 63, nw = blockDim.x >> 6, slots = topk + 1;
    int r = threadIdx.x >> 6;
    if (r >= rows) return;
    RouteIn<PER> cur, nxt;
    route_load<PER>(logits + (size_t)r * routed, routed, gate, cur);
    for (; r < rows; r += nw) {
        const int rn = r + nw < rows ? r + nw : r;
        route_load<PER>(logits + (size_t)rn * routed, routed, gate, nxt);
        int pick;
        float weight;
        route_pick<PER>(cur, logits + (size_t)r * routed, routed, topk, routed, pick, weight, gate);
        if (lane <= topk) {
            pk[r * slots + lane] = pick;
            wt[r * slots + lane] = weight;
        }
        cur = nxt;
    }
}


// route_group_kernel's work in one workgroup: wave w routes tokens w, w + waves, ... into LDS and global picks /
// weights, then the workgroup groups them (group_small_body) and writes the item plan. lds: route_group_lds bytes.
__device__ __forceinline__ void route_group_body(uint32_t* lds, int* scan_scratch, const float* __restrict__ logits,
                                                 int rows, int routed, int topk, int* __restrict__ picks,
                                                 float* __restrict__ weights, int* __restrict__ ids,
                                                 int* __restrict__ count, int* __restrict__ members, int maxm, int bm,
                                                 int* __restrict__ plan_ucnt, int* __restrict__ plan_items,
                                                 int* __restrict__ plan, int plan_E, RouteGate gate) {
    const int slots = topk + 1, E = routed + 1;
    int* pk = reinterpret_cast<int*>(lds);                     // [rows][slots]
    float* wt = reinterpret_cast<float*>(pk + rows * slots);   // [rows][slots]
    uint32_t* rest = reinterpret_cast<uint32_t*>(wt + rows * slots);
    if (routed <= 64) route_rows<1>(logits, rows, routed, topk, pk, wt, gate);
    else if (routed <= 128) route_rows<2>(logits, rows, routed, topk, pk, wt, gate);
    else if (routed <= 256) route_rows<4>(logits, rows, routed, topk, pk, wt, gate);
    else if (routed <= 320) route_rows<5>(logits, rows, routed, topk, pk, wt, gate);
    else if (routed <= 512) route_rows<8>(logits, rows, routed, topk, pk, wt, gate);
    else route_rows<ROUTE_MAX_E / 64>(logits, rows, routed, topk, pk, wt, gate);
    __syncthreads();
    for (int i = threadIdx.x; i < rows * slots; i += blockDim.x) {
        picks[i] = pk[i];
        weights[i] = wt[i];
    }
    group_small_body(pk, rows, slots, E, ids, count, members, maxm, rest, scan_scratch, bm, plan_ucnt, plan_items,
                     plan, plan_E);
}


// Launch 3, workgroup per expert (e; scan_scratch: 16 ints, 16-byte aligned; tot_sh: 4 ints, both LDS): its place among the used experts, ids / count, its members and its -1 tail. A
// thread per row: a member's position is the popcount prefix of its bitmap word plus the set bits below it in the
// word, so no thread walks an expert's rows in sequence. With `plan` (bm rows an item) it also writes the prefill
// engine's item plan, as prefill_plan_kernel would from the finished table: plan_ucnt[u] = members of used expert
// u, plan_items = (u << 16) | pass for the ceil(members / bm) passes of each u in u order, plan[0] = item count.
__device__ __forceinline__ void group_scatter_body(int e, int* scan_scratch, int* tot_sh, const int* __restrict__ picks,
                                                   int rows, int slots, int E, const uint32_t* __restrict__ bits,
                                                   const uint8_t* __restrict__ first, const int* __restrict__ prefix,
                                                   const int* __restrict__ counts, int* __restrict__ ids,
                                                   int* __restrict__ count, int* __restrict__ members, int maxm,
                                                   int bm, int* __restrict__ plan_ucnt, int* __restrict__ plan_items,
                                                   int* __restrict__ plan, int plan_E) {
    const int NWD = (rows + 31) >> 5;
    int below = 0, used = 0, ibelow = 0, itotal = 0;
    for (int q = threadIdx.x; q < E; q += blockDim.x) {
        const int c = counts[q], np = plan && q < plan_E ? (c + bm - 1) / bm : 0;
        used += c > 0;
        below += (q < e) & (c > 0);
        itotal += np;
        ibelow += q < e ? np : 0;
    }
    int t[4];
    block_scan(below, scan_scratch, &t[0]);
    block_scan(used, scan_scratch, &t[1]);
    if (plan) {
        block_scan(ibelow, scan_scratch, &t[2]);
        block_scan(itotal, scan_scratch, &t[3]);
    }
    if (threadIdx.x == 0)
        for (int i = 0; i < 4; ++i) tot_sh[i] = t[i];
    __syncthreads();
    below = tot_sh[0];
    used = tot_sh[1];
    const int ce = counts[e];
    if (e == 0 && threadIdx.x == 0) {
        *count = used;
        if (plan) plan[0] = tot_sh[3];
    }
    if (ce > 0) {
        const int u = below;
        if (threadIdx.x == 0) ids[u] = e;
        if (plan) {
            // experts at or above plan_E (a shared expert that is not EXL3) get no items
            const int np = e < plan_E ? (ce + bm - 1) / bm : 0, first = tot_sh[2];
            if (threadIdx.x == 0) plan_ucnt[u] = ce;
            for (int k = threadIdx.x; k < np; k += blockDim.x) plan_items[first + k] = (u << 16) | k;
        }
        // rows in batches of UB a thread: every load of a batch is issued before any of its values is used (the
        // empty asm keeps the compiler from sinking a load into the branch that uses it), so a batch costs one
        // round trip; first[] of a row outside the expert is loaded and never used
        constexpr int UB = 8;
        const uint32_t* be = bits + (size_t)e * NWD;
        const int* pe = prefix + (size_t)e * NWD;
        const uint8_t* fe = first + (size_t)e * rows;
        for (int r0 = threadIdx.x; r0 < rows; r0 += UB * blockDim.x) {
            uint32_t b[UB];
            int pos[UB], sl[UB];
#pragma unroll
            for (int k = 0; k < UB; ++k) {
                const int r = min(r0 + k * (int)blockDim.x, rows - 1);
                b[k] = be[r >> 5];
                pos[k] = pe[r >> 5];
                sl[k] = fe[r];
            }
#pragma unroll
            for (int k = 0; k < UB; ++k) __asm__ volatile("" : "+v"(b[k]), "+v"(pos[k]), "+v"(sl[k]));
#pragma unroll
            for (int k = 0; k < UB; ++k) {
                const int r = r0 + k * (int)blockDim.x;
                if (r < rows && ((b[k] >> (r & 31)) & 1u))
                    members[(size_t)u * maxm + pos[k] + __popc(b[k] & ((1u << (r & 31)) - 1u))] = r * 32 + sl[k];
            }
        }
        for (int j = ce + threadIdx.x; j < maxm; j += blockDim.x) members[(size_t)u * maxm + j] = -1;
    }
    // rows [used, E) of the table: owned by the workgroup with the same index (never a used row above)
    if (e >= used)
        for (int j = threadIdx.x; j < maxm; j += blockDim.x) members[(size_t)e * maxm + j] = -1;
}

}  // namespace gfr
