// Prefill-chunk experts on gfx950 (placeholder engine: scratch ownership; the MFMA kernels come next).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "exl3_format.hpp"
#include "launch.hpp"
#include "prefill.hpp"

struct gfr_fast_experts {
    gfr::PrefillDims d;
    uint16_t *xg, *xu, *xd;
    float* out;
};

namespace gfr {

hipError_t prefill_create(gfr_fast_experts** out, int hidden, int inter, int slots, int exl3_slots, int experts,
                          int max_rows) {
    gfr_fast_experts* fx = new gfr_fast_experts{{hidden, inter, slots, exl3_slots, experts, max_rows},
                                                nullptr, nullptr, nullptr, nullptr};
    const size_t P = (size_t)max_rows * slots;
    hipError_t e;
    if ((e = hipMalloc(&fx->xg, P * hidden * 2)) != hipSuccess || (e = hipMalloc(&fx->xu, P * hidden * 2)) != hipSuccess ||
        (e = hipMalloc(&fx->xd, P * inter * 2)) != hipSuccess || (e = hipMalloc(&fx->out, P * hidden * 4)) != hipSuccess) {
        prefill_destroy(fx);
        return e;
    }
    *out = fx;
    return hipSuccess;
}

PrefillDims prefill_dims(const gfr_fast_experts* fx) { return fx->d; }

hipError_t prefill_run(gfr_fast_experts*, hipStream_t, const gfr_exl3_experts*, const uint16_t*, int, const int*,
                       const int*, const int*, const int*, int, int, bool) {
    return hipErrorNotSupported;
}

float* prefill_output(const gfr_fast_experts* fx) { return fx->out; }
uint16_t* prefill_xd(const gfr_fast_experts* fx) { return fx->xd; }

void prefill_destroy(gfr_fast_experts* fx) {
    if (!fx) return;
    for (void* p : {(void*)fx->xg, (void*)fx->xu, (void*)fx->xd, (void*)fx->out})
        if (p) (void)hipFree(p);
    delete fx;
}

}  // namespace gfr
