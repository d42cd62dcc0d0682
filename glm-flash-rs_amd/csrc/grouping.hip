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
#include "grouping_body.hpp"

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

// Launch 3 (group_scatter_body), workgroup per expert.
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
    group_scatter_body(blockIdx.x, scan_scratch, tot_sh, picks, rows, slots, E, bits, first, prefix, counts, ids,
                       count, members, maxm, bm, plan_ucnt, plan_items, plan, plan_E);
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
                              int bm, int* plan_ucnt, int* plan_items, int* plan, int plan_E, bool scatter) {
    if ((size_t)E * 8 * 4 > GROUP_LDS_MAX) return hipErrorInvalidValue;
    group_mark_kernel<<<(rows + 255) / 256, 256, (size_t)E * 8 * 4, s>>>(picks, rows, slots, E, bits, first);
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return err;
    group_prefix_kernel<<<E, 256, 0, s>>>(bits, rows, prefix, counts);
    if ((err = hipGetLastError()) != hipSuccess) return err;
    if (!scatter) return hipSuccess;
    group_scatter_kernel<<<E, 256, 0, s>>>(picks, rows, slots, E, bits, first, prefix, counts, ids, count, members, maxm,
                                            bm, plan_ucnt, plan_items, plan, plan_E);
    return hipGetLastError();
}

}  // namespace gfr
