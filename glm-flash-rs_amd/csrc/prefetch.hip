// Cache-warming reads of weight memory for a decode round's idle windows: the reference's L2 prefetch library
// (native/l2-prefetch/l2pf.cu, bridge.cpp), on MI355X.
//
// A kernel here only reads weight memory and writes nothing, so it cannot change a bit of any result; it changes
// where the next kernels find their weights. gfx950 has no prefetch-to-L2 instruction like the bulk-copy unit the
// reference uses, so each lane loads one dword of a 128-byte line: the line is filled into the reading XCD's L2 and
// into the memory-side cache (MALL, 256 MB), which serves the expert launches on every XCD afterwards. A lane's loads
// and the wait for them are one asm statement with early-clobber outputs: the loaded registers are never read, and
// no register the compiler allocates can be written by a load still in flight.
//
// Two device entry points, as the reference's:
//   segments  a table of (address, bytes) pairs in device memory (a host-planned list of the next kernels' weights)
//   experts   device-indexed: the first `bytes` of every routed expert of a grouping (ids[0 .. count)) in the gate and
//             up trellis tensors (bases[0], bases[1] + id * stride), with no host round trip, so it can be captured
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/gfr_moe.h"

namespace gfr {
int set_error(int code, const std::string& msg);   // gfr_moe_api.hip (the thread's gfr_last_error)

constexpr uint64_t PF_LINE = 128;

// One dword of each 128-byte line of [p, p + bytes) for lines first, first + stride, ...; four lines a lane in flight
// (the lines past the end of a group re-read the group's first line). p is 16-byte aligned and bytes a multiple of 16.
__device__ __forceinline__ void touch_lines(const uint8_t* p, uint64_t bytes, uint64_t first, uint64_t stride) {
    const uint64_t lines = (bytes + PF_LINE - 1) / PF_LINE;
    for (uint64_t i = first; i < lines; i += 4 * stride) {
        const uint8_t* a[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint64_t l = i + k * stride;
            a[k] = p + (l < lines ? l : i) * PF_LINE;
        }
        uint32_t d0, d1, d2, d3;
        __asm__ volatile("global_load_dword %0, %4, off\n\tglobal_load_dword %1, %5, off\n\t"
                         "global_load_dword %2, %6, off\n\tglobal_load_dword %3, %7, off\n\t"
                         "s_waitcnt vmcnt(0)"
                         : "=&v"(d0), "=&v"(d1), "=&v"(d2), "=&v"(d3)
                         : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3])
                         : "memory");
    }
}

// table: n pairs of int64 (device address, bytes). Segment s starts at thread s mod the grid, so a table of many
// one-line segments spreads over the threads (l2pf.cu:58-70). Entries that are not 16-byte aligned, or empty, are
// skipped (the reference's host plan never produces them).
__global__ void __launch_bounds__(256) prefetch_segments_kernel(const int64_t* __restrict__ table, int n) {
    const uint64_t index = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (int s = 0; s < n; ++s) {
        const uint64_t addr = (uint64_t)table[2 * s];
        const int64_t bytes = table[2 * s + 1];
        if (addr == 0 || (addr & 15) || bytes <= 0 || (bytes & 15)) continue;
        const uint64_t first = (index + stride - (uint64_t)s % stride) % stride;
        touch_lines(reinterpret_cast<const uint8_t*>(addr), (uint64_t)bytes, first, stride);
    }
}

// The first `bytes` of expert ids[u] in each of the two matrices, for u < min(count[0], maxu): the (u, matrix) ranges
// are segments spread over the whole grid as in the segment kernel (range s starts at thread s), so a few experts
// still use every workgroup; ids outside [0, experts) are skipped, so no read leaves the expert tensors
// (l2pf.cu:72-88 gives each expert one block; the work is the same).
__global__ void __launch_bounds__(256) prefetch_experts_kernel(const int32_t* __restrict__ ids,
                                                              const int32_t* __restrict__ count, int maxu,
                                                              const int64_t* __restrict__ bases, int64_t stride,
                                                              int64_t bytes, int64_t experts) {
    const uint64_t index = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
    const int c = *count, n = c < maxu ? c : maxu;
    for (int s = 0; s < 2 * n; ++s) {
        const int64_t e = ids[s >> 1];
        if (e < 0 || e >= experts) continue;
        const uint8_t* p = reinterpret_cast<const uint8_t*>((uint64_t)bases[s & 1]) + e * stride;
        touch_lines(p, (uint64_t)bytes, (index + nthreads - (uint64_t)s % nthreads) % nthreads, nthreads);
    }
}

}  // namespace gfr

namespace {
int einval(const char* what) { return gfr::set_error(GFR_EINVAL, what); }
int hip_err(hipError_t e, const char* what) {
    return gfr::set_error((int)e, std::string("HIP ") + hipGetErrorName(e) + ": " + hipGetErrorString(e) + " (" +
                                      what + ")");
}
}  // namespace

extern "C" {

uint32_t gfr_prefetch_abi(void) { return 1; }

int gfr_prefetch_properties(int* cus, int* l2_bytes) {
    if (!cus || !l2_bytes) return einval("null output");
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_err(e, "hipGetDevice");
    if ((e = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev)) != hipSuccess)
        return hip_err(e, "CU count");
    if ((e = hipDeviceGetAttribute(l2_bytes, hipDeviceAttributeL2CacheSize, dev)) != hipSuccess)
        return hip_err(e, "L2 size");
    return 0;
}

int gfr_prefetch_capturing(hipStream_t stream, int* active) {
    if (!stream || !active) return einval("null stream or output");
    hipStreamCaptureStatus st;
    const hipError_t e = hipStreamIsCapturing(stream, &st);
    if (e != hipSuccess) return hip_err(e, "hipStreamIsCapturing");
    if (st == hipStreamCaptureStatusInvalidated) return hip_err(hipErrorStreamCaptureInvalidated, "capture");
    *active = st == hipStreamCaptureStatusActive;
    return 0;
}

int gfr_prefetch_segments(const int64_t* table, int count, int grid, hipStream_t stream) {
    if (!table || count <= 0 || grid <= 0 || !stream) return einval("prefetch segments: null table / stream, or count / grid <= 0");
    gfr::prefetch_segments_kernel<<<grid, 128, 0, stream>>>(table, count);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_err(e, "prefetch segments launch");
}

int gfr_prefetch_experts(const int32_t* ids, const int32_t* count, int maxu, const int64_t* bases, int64_t stride,
                         int64_t bytes, int64_t experts, int grid, hipStream_t stream) {
    if (!ids || !count || !bases || maxu <= 0 || experts <= 0 || stride <= 0 || bytes <= 0 || bytes > stride ||
        bytes > GFR_PREFETCH_EXPERT_BYTES_MAX || bytes % 16 || stride % 16 || grid <= 0 || !stream)
        return einval("prefetch experts: bounds (bytes in (0, min(stride, 64 KiB)], multiples of 16, grid > 0)");
    gfr::prefetch_experts_kernel<<<grid, 128, 0, stream>>>(ids, count, maxu, bases, stride, bytes, experts);
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? 0 : hip_err(e, "prefetch experts launch");
}

}  // extern "C"
