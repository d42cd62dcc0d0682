// Token -> expert bucketing on gfx950, bit-exact to glm-flash-rs native/grouping.cu (group_clear/mark/prefix/ids/
// scatter and group_small) and to the host oracle of src/grouping.rs:141-192.
//
// Output contract (grouping.rs:12-112): count = number of distinct experts in picks[rows][slots]; ids[u] = the u-th
// smallest of them; members[u * maxm + i] = the codes r * 32 + slot of expert ids[u], rows ascending (a row counts
// once, with the first slot that holds the expert), then -1 up to maxm; members rows u in [count, E) are all -1.
// The order never depends on atomic arrival: rows are marked in a bitmap (atomicOr is order-free) and read back
// in bit order.
//
// Two paths: rows <= GROUP_SMALL_ROWS (launch.hpp) runs in one 1024-thread workgroup with the bitmap in LDS; larger windows run three
// launches (per-256-row LDS bitmaps, per-expert popcount prefix, per-expert scatter), which also lifts the
// reference's 8192-row limit.
#include "group_small.hpp"

namespace gfr {

__global__ void __launch_bounds__(1024) group_small_kernel(const int* __restrict__ picks, int rows, int slots,
                                                           int E, int* __restrict__ ids, int* __restrict__ count,
                                                           int* __restrict__ members, int maxm) {
    extern __shared__ uint32_t lds[];
    __shared__ __attribute__((aligned(16))) int scan_scratch[16];
    int* pk = reinterpret_cast<int*>(lds);                     // [rows][slots], read many times below
    for (int i = threadIdx.x; i < rows * slots; i += blockDim.x) pk[i] = picks[i];
    __syncthreads();
    group_small_body(pk, rows, slots, E, ids, count, members, maxm, lds + rows * slots, scan_scratch);
}

// Decode windows in one launch: route_group_body in one 1024-thread workgroup. rows <= GROUP_SMALL_ROWS.
__global__ void __launch_bounds__(1024) route_group_kernel(const float* __restrict__ logits, int rows, int routed,
                                                           int topk, int* __restrict__ picks,
                                                           float* __restrict__ weights, int* __restrict__ ids,
                                                           int* __restrict__ count, int* __restrict__ members,
                                                           int maxm, int bm, int* __restrict__ plan_ucnt,
                                                           int* __restrict__ plan_items, int* __restrict__ plan,
                                                           int plan_E, RouteGate gate) {
    extern __shared__ uint32_t lds[];
    __shared__ __attribute__((aligned(16))) int scan_scratch[16];
    route_group_body(lds, scan_scratch, logits, rows, routed, topk, picks, weights, ids, count, members, maxm, bm,
                     plan_ucnt, plan_items, plan, plan_E, gate);
}

// Large windows, launch 1: the 256 rows of this workgroup marked in an LDS bitmap [E][8], stored to
// bits[e][NWD] (each global word is owned by exactly one workgroup, so no clear launch is needed), and
// first[e][r] = the first slot of row r that holds e (the slots stored last to first, so the first one stays).
__global__ void __launch_bounds__(256) group_mark_kernel(const int* __restrict__ picks, int rows, int slots, int E,
                                                         uint32_t* __restrict__ bits, uint8_t* __restrict__ first) {
    extern __shared__ uint32_t lb[];                         // [E][8]
    const int NWD = (rows + 31) >> 5;
    for (int i = threadIdx.x; i < E * 8; i += blockDim.x) lb[i] = 0;
    __syncthreads();
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r < rows)
        for (int s = slots - 1; s >= 0; --s) {
            const int e = picks[r * slots + s];
            if (e >= 0 && e < E) {
                atomicOr(&lb[e * 8 + (threadIdx.x >> 5)], 1u << (r & 31));
                first[(size_t)e * rows + r] = (uint8_t)s;
            }
        }
    __syncthreads();
    for (int i = threadIdx.x; i < E * 8; i += blockDim.x) {
        const int e = i >> 3, w = blockIdx.x * 8 + (i & 7);
        if (w < NWD) bits[(size_t)e * NWD + w] = lb[i];
    }
}

// Launch 2, workgroup per expert: exclusive popcount prefix of its bitmap words, and its row count.
__global__ void __launch_bounds__(256) group_prefix_kernel(const uint32_t* __restrict__ bits, int rows,
                                                           int* __restrict__ prefix, int* __restrict__ counts) {
    __shared__ __attribute__((aligned(16))) int scan_scratch[16];
    const int e = blockIdx.x, NWD = (rows + 31) >> 5;
    const int per = (NWD + blockDim.x - 1) / blockDim.x, w0 = threadIdx.x * per;
    const uint32_t* b = bits + (size_t)e * NWD;
    int c = 0;
    for (int w = w0; w < w0 + per && w < NWD; ++w) c += __popc(b[w]);
    int total;
    int run = block_scan(c, scan_scratch, &total) - c;
    for (int w = w0; w < w0 + per && w < NWD; ++w) {
        prefix[(size_t)e * NWD + w] = run;
        run += __popc(b[w]);
    }
    if (threadIdx.x == 0) counts[e] = total;
}

// Launch 3, workgroup per expert: its place among the used experts, ids / count, its members and its -1 tail. A
// thread per row: a member's position is the popcount prefix of its bitmap word plus the set bits below it in the
// word, so no thread walks an expert's rows in sequence. With `plan` (bm rows an item) it also writes the prefill
// engine's item plan, as prefill_plan_kernel would from the finished table: plan_ucnt[u] = members of used expert
// u, plan_items = (u << 16) | pass for the ceil(members / bm) passes of each u in u order, plan[0] = item count.
__global__ void __launch_bounds__(256) group_scatter_kernel(const int* __restrict__ picks, int rows, int slots,
                                                            int E, const uint32_t* __restrict__ bits,
                                                            const uint8_t* __restrict__ first,
                                                            const int* __restrict__ prefix,
                                                            const int* __restrict__ counts, int* __restrict__ ids,
                                                            int* __restrict__ count, int* __restrict__ members,
                                                            int maxm, int bm, int* __restrict__ plan_ucnt,
                                                            int* __restrict__ plan_items, int* __restrict__ plan,
                                                            int plan_E) {
    __shared__ __attribute__((aligned(16))) int scan_scratch[16];
    __shared__ int tot_sh[4];
    const int e = blockIdx.x, NWD = (rows + 31) >> 5;
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

#include "launch.hpp"

namespace gfr {

size_t group_small_lds(int rows, int slots, int E) {
    return ((size_t)rows * slots + (size_t)E * ((rows + 31) / 32) + 2 * (size_t)E) * 4;
}
hipError_t launch_group_small(hipStream_t s, const int* picks, int rows, int slots, int E, int* ids, int* count,
                              int* members, int maxm) {
    const size_t lds = group_small_lds(rows, slots, E);
    if (lds > GROUP_LDS_MAX) return hipErrorInvalidValue;
    group_small_kernel<<<1, 1024, lds, s>>>(picks, rows, slots, E, ids, count, members, maxm);
    return hipGetLastError();
}

size_t route_group_lds(int rows, int slots, int E) {
    return (2 * (size_t)rows * slots + (size_t)E * ((rows + 31) / 32) + 2 * (size_t)E) * 4;
}

hipError_t launch_route_group(hipStream_t s, const float* logits, int rows, int routed, int topk, int* picks,
                              float* weights, int* ids, int* count, int* members, int maxm, int bm, int* plan_ucnt,
                              int* plan_items, int* plan, int plan_E, const float* bias, float scale) {
    const int E = routed + 1, slots = topk + 1;
    const size_t lds = route_group_lds(rows, slots, E);
    if (lds > GROUP_LDS_MAX) return hipErrorInvalidValue;
    route_group_kernel<<<1, 1024, lds, s>>>(logits, rows, routed, topk, picks, weights, ids, count, members, maxm,
                                            bm, plan_ucnt, plan_items, plan, plan_E, RouteGate{bias, scale});
    return hipGetLastError();
}

hipError_t launch_group_large(hipStream_t s, const int* picks, int rows, int slots, int E, uint32_t* bits,
                              uint8_t* first, int* prefix, int* counts, int* ids, int* count, int* members, int maxm,
                              int bm, int* plan_ucnt, int* plan_items, int* plan, int plan_E) {
    if ((size_t)E * 8 * 4 > GROUP_LDS_MAX) return hipErrorInvalidValue;
    group_mark_kernel<<<(rows + 255) / 256, 256, (size_t)E * 8 * 4, s>>>(picks, rows, slots, E, bits, first);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    group_prefix_kernel<<<E, 256, 0, s>>>(bits, rows, prefix, counts);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    group_scatter_kernel<<<E, 256, 0, s>>>(picks, rows, slots, E, bits, first, prefix, counts, ids, count, members, maxm,
                                            bm, plan_ucnt, plan_items, plan, plan_E);
    return hipGetLastError();
}

}  // namespace gfr
