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
//             up trellis tensors (at bases[m] + id * stride, m = 0, 1), with no host round trip, so it can be captured
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string>

#include "../../include/gfr_moe.h"

namespace gfr {
int set_error(int code, const std::string& msg);   // gfr_moe_api.hip (the thread's gfr_last_error)

constexpr uint64_t PF_LINE = 128;

// Four line reads of one lane, issued together and waited for together (one memory round trip). The loaded registers
// are never read; the outputs are early-clobber so that no register the compiler allocates (an address of the next
// batch) can be written by a load still in flight.
__device__ __forceinline__ void touch4(const uint8_t* a0, const uint8_t* a1, const uint8_t* a2, const uint8_t* a3) {
    uint32_t d0, d1, d2, d3;
    __asm__ volatile("global_load_dword %0, %4, off\n\tglobal_load_dword %1, %5, off\n\t"
                     "global_load_dword %2, %6, off\n\tglobal_load_dword %3, %7, off\n\t"
                     "s_waitcnt vmcnt(0)"
                     : "=&v"(d0), "=&v"(d1), "=&v"(d2), "=&v"(d3)
                     : "v"(a0), "v"(a1), "v"(a2), "v"(a3)
                     : "memory");
}

// A lane's line addresses, gathered over every range before any is read: four make one round trip, whichever
// ranges they come from (a lane waits once per four lines, not once per range). A partial batch repeats its first
// address.
struct LineBatch {
    const uint8_t* a[4];
    int n = 0;
    __device__ __forceinline__ void add(const uint8_t* p) {
        a[n++] = p;
        if (n == 4) {
            touch4(a[0], a[1], a[2], a[3]);
            n = 0;
        }
    }
    __device__ __forceinline__ void flush() {
        if (n == 0) return;
        for (int k = n; k < 4; ++k) a[k] = a[0];
        touch4(a[0], a[1], a[2], a[3]);
        n = 0;
    }
};

// table: n pairs of int64 (device address, bytes). The ranges' 128-byte lines are numbered in table order and
// thread t of the grid reads lines t, t + threads, ... (one dword a line). Entries that are not 16-byte aligned, or
// empty, are skipped (the reference's host plan never produces them). l2pf.cu:58-70 instead hands each segment to
// every thread in turn, which here would cost one round trip a segment.
__global__ void __launch_bounds__(256) prefetch_segments_kernel(const int64_t* __restrict__ table, int n) {
    const uint64_t index = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    LineBatch lb;
    uint64_t pos = index, start = 0;                   // this thread's next line, the current range's first line
    for (int s = 0; s < n; ++s) {
        const uint64_t addr = (uint64_t)table[2 * s];
        const int64_t bytes = table[2 * s + 1];
        if (addr == 0 || (addr & 15) || bytes <= 0 || (bytes & 15)) continue;
        const uint64_t lines = ((uint64_t)bytes + PF_LINE - 1) / PF_LINE;
        for (; pos < start + lines; pos += stride) lb.add(reinterpret_cast<const uint8_t*>(addr) + (pos - start) * PF_LINE);
        start += lines;
    }
    lb.flush();
}

// The first `bytes` of expert ids[u] in each of the two matrices, for u < min(count[0], maxu): the ranges
// (u, matrix) are numbered u-major and their lines read as in the segment kernel; ids outside [0, experts) are
// skipped, so no read leaves the expert tensors (l2pf.cu:72-88 gives each expert one block instead).
__global__ void __launch_bounds__(256) prefetch_experts_kernel(const int32_t* __restrict__ ids,
                                                              const int32_t* __restrict__ count, int maxu,
                                                              const int64_t* __restrict__ bases, int64_t stride,
                                                              int64_t bytes, int64_t experts) {
    const uint64_t index = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const uint64_t nthreads = (uint64_t)gridDim.x * blockDim.x;
    const int c = *count, n = c < maxu ? c : maxu;
    const uint64_t lines = ((uint64_t)bytes + PF_LINE - 1) / PF_LINE;
    LineBatch lb;
    for (uint64_t pos = index; pos < 2 * (uint64_t)n * lines; pos += nthreads) {
        const uint64_t s = pos / lines, l = pos - s * lines;
        const int64_t e = ids[s >> 1];
        if (e < 0 || e >= experts) continue;
        lb.add(reinterpret_cast<const uint8_t*>((uint64_t)bases[s & 1]) + e * stride + l * PF_LINE);
    }
    lb.flush();
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
