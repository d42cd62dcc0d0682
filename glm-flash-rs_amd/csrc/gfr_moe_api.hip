// The C ABI of include/gfr_moe.h: engines that own scratch (allocated once, zeroed) and issue the gfx950 kernels
// on the caller's stream. Mirrors the reference's Rust owners (grouping.rs, experts.rs, fast_experts.rs, moe.rs):
// same buffer contracts, same precondition checks, no allocation / free / host sync inside run.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>
#include <stdint.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <mutex>
#include <string>

#include "../../include/gfr_moe.h"
#include "launch.hpp"
#include "prefill.hpp"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

// hipError_t -> the reference's "CUDA {code} {name}: {msg}" shape (cuda.rs:102-123)
int hip_fail(hipError_t e, const char* what) {
    return fail((int)e, "HIP %d %s: %s (%s)", (int)e, hipGetErrorName(e), hipGetErrorString(e), what);
}


template <typename T>
int alloc_zero(T** p, size_t count, const char* what) {
    *p = nullptr;
    if (count == 0) count = 1;
    hipError_t e = hipMalloc((void**)p, count * sizeof(T));
    if (e != hipSuccess) return hip_fail(e, what);
    e = hipMemset(*p, 0, count * sizeof(T));
    if (e != hipSuccess) return hip_fail(e, what);
    return 0;
}

void free_all(std::initializer_list<void*> ps) {
    for (void* p : ps)
        if (p) (void)hipFree(p);
}

int check_weights(const gfr_exl3_experts* w, int hidden, int inter) {
    if (!w) return fail(GFR_EINVAL, "null weights");
    if (w->hidden != hidden || w->inter != inter)
        return fail(GFR_EINVAL, "weights shape %dx%d, engine %dx%d", w->hidden, w->inter, hidden, inter);
    if (w->bits < 2 || w->bits > 5) return fail(GFR_EINVAL, "bits %d outside 2..5", w->bits);
    if (w->experts <= 0) return fail(GFR_EINVAL, "experts %d", w->experts);
    if (!w->gt || !w->ut || !w->dt || !w->suh_g || !w->suh_u || !w->suh_d || !w->svh_g || !w->svh_u || !w->svh_d)
        return fail(GFR_EINVAL, "null weight tensor");
    return 0;
}

int check_shape(int hidden, int inter) {
    if (hidden <= 0 || inter <= 0 || hidden % 128 || inter % 128)
        return fail(GFR_EINVAL, "hidden %d / inter %d must be positive multiples of 128", hidden, inter);
    if (hidden % 256 || inter % 256)
        return fail(GFR_EINVAL, "hidden %d / inter %d must be multiples of 256 (k split of the GEMV)", hidden, inter);
    if (hidden / 128 > 4096 || inter / 128 > 4096) return fail(GFR_EINVAL, "hidden / inter too large");
    return 0;
}

}  // namespace

namespace gfr {
// the thread's last error, for the other translation units of the library (prepared.hip)
int set_error(int code, const std::string& msg) { return fail(code, "%s", msg.c_str()); }
}  // namespace gfr

struct gfr_grouping {
    int experts, slots, max_rows;
    uint32_t* bits;
    int *prefix, *counts, *ids, *count, *members;
    uint8_t* first;            // [experts][max_rows]: the first slot of row r that holds expert e (large windows)
};

struct gfr_experts {
    int hidden, inter, slots, exl3_slots, max_rows;
    uint16_t* xd;
    float *zgu, *zd, *y;             // gate/up and down split partials, expert outputs
};

struct gfr_linear {
    int kin, n, bits;
    int *pick, *ids, *count, *members;
    float* z;
};

struct gfr_moe {
    int hidden, inter, routed, topk, slots, max_rows, decode_rows;
    float* weights;
    int* picks;
    float* out;
    gfr_grouping* group_dec;   // member stride = the decode engine's bound
    gfr_grouping* group_pre;   // member stride = max_rows (prefill chunks)
    gfr_experts* dec;
    gfr_fast_experts* pre;
    const float* route_bias;   // the router's gate (gfr_moe_set_router): nullptr = softmax
    float route_scale;
    int shared_exl3;           // 1: the shared expert is EXL3 (weights hold routed + 1 experts); 0: its output is the
                               // caller's (gfr_moe_run_shared), weights hold the routed experts only
    float* logits;             // [max_rows][routed] router logits of gfr_moe_run_router
    int launches;              // measurement: rows == 1 issues only the first `launches` launches (0: all)
    gfr_shared_fp8* sfp8;      // shared_exl3 = 0: the FP8 shared expert's engine and output [max_rows][hidden]
    float* shared_out;
};

struct gfr_shared_fp8 {
    int hidden, inter, max_rows;
    uint16_t* gu;    // [max_rows][2 inter] bf16
    uint16_t* act;   // [max_rows][inter] bf16
    rocblas_handle blas;   // the prefill form's GEMMs, with a workspace of its own (no allocation at run)
    void* blas_ws;
};

extern "C" {

const char* gfr_last_error(void) { return g_last_error.c_str(); }
const char* gfr_version(void) { return "gfr_moe 0.1 gfx950"; }

// ---- grouping ---------------------------------------------------------------------------------------------------
int gfr_grouping_create(gfr_grouping** out, int experts, int slots, int max_rows) {
    if (!out) return fail(GFR_EINVAL, "null out");
    *out = nullptr;
    // the large path keeps an 8-word bitmap row per expert in LDS (64 KiB at 2048 experts)
    if (experts <= 0 || experts > 2048) return fail(GFR_EINVAL, "grouping experts %d outside 1..2048", experts);
    if (slots <= 0 || slots > 32) return fail(GFR_EINVAL, "grouping slots %d outside 1..32", slots);
    if (max_rows <= 0 || max_rows > (1 << 20)) return fail(GFR_EINVAL, "grouping capacity %d", max_rows);
    gfr_grouping* g = new gfr_grouping{experts, slots, max_rows, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    const size_t nwd = (size_t)(max_rows + 31) / 32;
    int rc;
    if ((rc = alloc_zero(&g->bits, (size_t)experts * nwd, "grouping bits")) ||
        (rc = alloc_zero(&g->prefix, (size_t)experts * nwd, "grouping prefix")) ||
        (rc = alloc_zero(&g->first, (size_t)experts * max_rows, "grouping first slots")) ||
        (rc = alloc_zero(&g->counts, (size_t)experts, "grouping counts")) ||
        (rc = alloc_zero(&g->ids, (size_t)experts, "grouping ids")) || (rc = alloc_zero(&g->count, 1, "count")) ||
        (rc = alloc_zero(&g->members, (size_t)experts * max_rows, "grouping members"))) {
        gfr_grouping_destroy(g);
        return rc;
    }
    *out = g;
    return 0;
}

int gfr_grouping_run(gfr_grouping* g, hipStream_t stream, const int32_t* picks, int rows) {
    if (!g || !picks) return fail(GFR_EINVAL, "null grouping or picks");
    if (rows <= 0 || rows > g->max_rows) return fail(GFR_EINVAL, "grouping rows %d exceed scratch %d", rows, g->max_rows);
    hipError_t e;
    if (rows <= gfr::GROUP_SMALL_ROWS && g->experts <= 1024 &&
        gfr::group_small_lds(rows, g->slots, g->experts) <= gfr::GROUP_LDS_MAX)
        e = gfr::launch_group_small(stream, picks, rows, g->slots, g->experts, g->ids, g->count, g->members,
                                    g->max_rows);
    else
        e = gfr::launch_group_large(stream, picks, rows, g->slots, g->experts, g->bits, g->first, g->prefix, g->counts,
                                    g->ids, g->count, g->members, g->max_rows);
    if (e != hipSuccess) return hip_fail(e, "grouping launch");
    return 0;
}

int32_t* gfr_grouping_ids(const gfr_grouping* g) { return g ? g->ids : nullptr; }
int32_t* gfr_grouping_count(const gfr_grouping* g) { return g ? g->count : nullptr; }
int32_t* gfr_grouping_members(const gfr_grouping* g) { return g ? g->members : nullptr; }

int gfr_grouping_destroy(gfr_grouping* g) {
    if (!g) return 0;
    free_all({g->bits, g->prefix, g->counts, g->ids, g->count, g->members, g->first});
    delete g;
    return 0;
}

// ---- decode / verify experts ------------------------------------------------------------------------------------
namespace {
// The decode launches: gate/up GEMV (+ rotation), down GEMV (+ gate/up epilogue), down epilogue (+ combine).
int experts_run(gfr_experts* ex, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                int input_stride, const int32_t* picks, const int32_t* ids, const int32_t* count,
                const int32_t* members, int rows, int maxm, const float* weights, float* out,
                const gfr::RouteOne* route = nullptr, const float* shared = nullptr, int shared_stride = 0,
                int launches = 0, hipEvent_t shared_ready = nullptr, const gfr::Fp8Shared* fp8 = nullptr) {
    const int P = rows * ex->slots, D = ex->hidden, N = ex->inter;
    const int maxu = P < w->experts ? P : w->experts;
    hipError_t e;
    if ((e = gfr::launch_expert_gateup(stream, input, input_stride, w->suh_g, w->suh_u, w->gt, w->ut, ids, count,
                                       members, ex->zgu, D, N, P, rows, maxm, ex->slots, w->experts, w->bits, maxu,
                                       route, w->dt, fp8)) !=
        hipSuccess)
        return hip_fail(e, "gate/up gemv");
    if (launches == 1) return 0;
    const int skgu = gfr::gemv_gateup_splits(D);
    if ((e = gfr::launch_expert_down(stream, ex->zgu, D, skgu, w->svh_g, w->svh_u, w->suh_d, 10.f, ex->xd, w->dt,
                                     w->svh_d,
                                     ids, count, members, ex->zd, N, P, rows, maxm, ex->slots, w->experts, w->bits,
                                     maxu, route, fp8)) != hipSuccess)
        return hip_fail(e, "down gemv");
    if (launches == 2) return 0;
    // the shared branch joins here: only the finish (down epilogue + combine) reads its output
    if (shared_ready && (e = hipStreamWaitEvent(stream, shared_ready, 0)) != hipSuccess)
        return hip_fail(e, "wait for the shared expert");
    if ((e = gfr::launch_sum_finish(stream, ex->zd, ex->y, rows, P, D, gfr::gemv_down_splits(N), ex->slots,
                                    ex->exl3_slots, weights, shared, shared_stride, out)) != hipSuccess)
        return hip_fail(e, "down epilogue");
    return 0;
}
}  // namespace

int gfr_experts_create(gfr_experts** out, int hidden, int inter, int slots, int exl3_slots, int max_rows) {
    if (!out) return fail(GFR_EINVAL, "null out");
    *out = nullptr;
    int rc = check_shape(hidden, inter);
    if (rc) return rc;
    if (slots <= 0 || slots > 32 || exl3_slots < 0 || exl3_slots > slots)
        return fail(GFR_EINVAL, "slots %d / exl3_slots %d", slots, exl3_slots);
    if (max_rows <= 0 || max_rows > 64) return fail(GFR_EINVAL, "expert verifier scratch bound: max_rows %d", max_rows);
    gfr_experts* ex = new gfr_experts{hidden, inter, slots, exl3_slots, max_rows, nullptr, nullptr, nullptr,
                                      nullptr};
    const size_t P = (size_t)max_rows * slots;
    const size_t zgu = 2 * (size_t)gfr::gemv_gateup_splits(hidden) * P * inter;
    const size_t zd = (size_t)gfr::gemv_down_splits(inter) * P * hidden;
    if ((rc = alloc_zero(&ex->xd, P * inter, "experts xd")) || (rc = alloc_zero(&ex->zgu, zgu, "experts zgu")) ||
        (rc = alloc_zero(&ex->zd, zd, "experts zd")) || (rc = alloc_zero(&ex->y, P * hidden, "experts y"))) {
        gfr_experts_destroy(ex);
        return rc;
    }
    *out = ex;
    return 0;
}

int gfr_experts_run_rows(gfr_experts* ex, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                         int input_stride, const int32_t* picks, const int32_t* ids, const int32_t* count,
                         const int32_t* members, int rows, int maxm) {
    if (!ex) return fail(GFR_EINVAL, "null experts");
    int rc = check_weights(w, ex->hidden, ex->inter);
    if (rc) return rc;
    if (!(rows > 0 && rows <= ex->max_rows && maxm >= rows && maxm <= ex->max_rows))
        return fail(GFR_EINVAL, "expert verifier row/member bounds: rows %d maxm %d max_rows %d", rows, maxm,
                    ex->max_rows);
    if (!input || !picks || !ids || !count || !members) return fail(GFR_EINVAL, "null input");
    if (input_stride < ex->hidden) return fail(GFR_EINVAL, "input stride %d < hidden %d", input_stride, ex->hidden);
    return experts_run(ex, stream, w, input, input_stride, picks, ids, count, members, rows, maxm, nullptr, nullptr);
}

float* gfr_experts_y(const gfr_experts* ex) { return ex ? ex->y : nullptr; }
uint16_t* gfr_experts_xd(const gfr_experts* ex) { return ex ? ex->xd : nullptr; }

int gfr_experts_destroy(gfr_experts* ex) {
    if (!ex) return 0;
    free_all({ex->xd, ex->zgu, ex->zd, ex->y});
    delete ex;
    return 0;
}

// ---- single linear ----------------------------------------------------------------------------------------------
int gfr_linear_create(gfr_linear** out, int kin, int n, int bits) {
    if (!out) return fail(GFR_EINVAL, "null out");
    *out = nullptr;
    int rc = check_shape(kin, n);
    if (rc) return rc;
    if (bits < 2 || bits > 5) return fail(GFR_EINVAL, "bits %d outside 2..5", bits);
    gfr_linear* l = new gfr_linear{kin, n, bits, nullptr, nullptr, nullptr, nullptr, nullptr};
    if ((rc = alloc_zero(&l->pick, 1, "linear pick")) || (rc = alloc_zero(&l->ids, 1, "linear ids")) ||
        (rc = alloc_zero(&l->count, 1, "linear count")) || (rc = alloc_zero(&l->members, 1, "linear members")) ||
        (rc = alloc_zero(&l->z, (size_t)gfr::gemv_linear_splits(kin) * n, "linear z"))) {
        gfr_linear_destroy(l);
        return rc;
    }
    const int one = 1;  // one expert (id 0, already zero), one member: row 0 slot 0 (code 0, already zero)
    hipError_t e = hipMemcpy(l->count, &one, sizeof one, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        gfr_linear_destroy(l);
        return hip_fail(e, "linear init");
    }
    *out = l;
    return 0;
}

int gfr_linear_run(gfr_linear* l, hipStream_t stream, const uint16_t* x, const uint32_t* trellis, const uint16_t* suh,
                   const uint16_t* svh, float* y) {
    if (!l || !x || !trellis || !suh || !svh || !y) return fail(GFR_EINVAL, "null argument");
    hipError_t e;
    // two launches: the GEMV with the input rotation fused (rot_in's arithmetic, exl3.cu:224-241), then the
    // ordered split sum, transform and output scale (down_epilogue_kernel)
    if ((e = gfr::launch_linear_fused(stream, x, suh, trellis, l->ids, l->count, l->members, l->z, l->kin, l->n,
                                      l->bits)) != hipSuccess)
        return hip_fail(e, "linear gemv");
    if ((e = gfr::launch_down_epilogue(stream, l->z, l->pick, svh, y, 1, l->n, gfr::gemv_linear_splits(l->kin), 1,
                                       1)) != hipSuccess)
        return hip_fail(e, "linear epilogue");
    return 0;
}

int gfr_linear_destroy(gfr_linear* l) {
    if (!l) return 0;
    free_all({l->pick, l->ids, l->count, l->members, l->z});
    delete l;
    return 0;
}

// ---- grouped GEMV alone ---------------------------------------------------------------------------------------
int gfr_exl3_gemv_splits(int kin) {
    if (kin <= 0 || kin % 64) return fail(GFR_EINVAL, "kin %d not a positive multiple of 64", kin);
    return gfr::gemv_splits(kin);
}

int gfr_exl3_grouped_gemv(hipStream_t stream, const uint16_t* x0, const uint16_t* x1, const uint32_t* t0,
                          const uint32_t* t1, const int32_t* uids, const int32_t* ucount, const int32_t* members,
                          float* z, int kin, int n, int pairs, int maxm, int slots, int experts, int bits, int mats,
                          int maxu) {
    if (!x0 || !t0 || !uids || !ucount || !members || !z || (mats == 2 && (!x1 || !t1)))
        return fail(GFR_EINVAL, "null argument");
    if (kin <= 0 || kin % 64 || n <= 0 || n % 128) return fail(GFR_EINVAL, "kin %d / n %d", kin, n);
    if (bits < 2 || bits > 5 || (mats != 1 && mats != 2)) return fail(GFR_EINVAL, "bits %d / mats %d", bits, mats);
    if (pairs <= 0 || maxm <= 0 || slots <= 0 || slots > 32 || experts <= 0 || maxu <= 0)
        return fail(GFR_EINVAL, "pairs %d maxm %d slots %d experts %d maxu %d", pairs, maxm, slots, experts, maxu);
    if (maxm > 64) return fail(GFR_EINVAL, "maxm %d: an expert's members are read one a lane (at most 64)", maxm);
    hipError_t e = gfr::launch_gemv(stream, x0, x1 ? x1 : x0, t0, t1 ? t1 : t0, uids, ucount, members, z, kin, n,
                                    pairs, maxm, slots, experts, bits, mats, maxu);
    if (e != hipSuccess) return hip_fail(e, "grouped gemv");
    return 0;
}

// ---- router alone -----------------------------------------------------------------------------------------------
int gfr_route_topk(hipStream_t stream, const float* logits, int rows, int routed, int topk, int32_t* picks,
                   float* weights) {
    if (!logits || !picks || !weights) return fail(GFR_EINVAL, "null argument");
    if (rows <= 0 || routed <= 0 || routed > 1024 || topk <= 0 || topk > 31 || topk > routed)
        return fail(GFR_EINVAL, "rows %d routed %d topk %d", rows, routed, topk);
    hipError_t e = gfr::launch_route(stream, logits, rows, routed, topk, routed, picks, weights);
    if (e != hipSuccess) return hip_fail(e, "route");
    return 0;
}

int gfr_route_topk_biased(hipStream_t stream, const float* logits, const float* bias, float scale, int rows,
                          int routed, int topk, int32_t* picks, float* weights) {
    if (!logits || !bias || !picks || !weights) return fail(GFR_EINVAL, "null argument");
    if (rows <= 0 || routed <= 0 || routed > 1024 || topk <= 0 || topk > 31 || topk > routed)
        return fail(GFR_EINVAL, "rows %d routed %d topk %d", rows, routed, topk);
    if (!(scale > 0.f)) return fail(GFR_EINVAL, "router scale %g must be positive", (double)scale);
    hipError_t e = gfr::launch_route(stream, logits, rows, routed, topk, routed, picks, weights, bias, scale);
    if (e != hipSuccess) return hip_fail(e, "route");
    return 0;
}

// ---- debug rotation ---------------------------------------------------------------------------------------------
int gfr_exl3_rotate(hipStream_t stream, const uint16_t* x, int x_stride, int x_f16, const int32_t* expert,
                    const uint16_t* suh, int k, int rows, uint16_t* out) {
    if (!x || !expert || !suh || !out) return fail(GFR_EINVAL, "null argument");
    if (k <= 0 || k % 128 || rows <= 0 || x_stride < k) return fail(GFR_EINVAL, "k %d rows %d stride %d", k, rows, x_stride);
    hipError_t e = gfr::launch_rot_in(stream, x, x_stride, x_f16 != 0, expert, suh, suh, out, out, k, rows, 1, 1, 1);
    if (e != hipSuccess) return hip_fail(e, "rotate");
    return 0;
}

// ---- debug decode -----------------------------------------------------------------------------------------------
int gfr_exl3_decode_tiles(hipStream_t stream, const uint32_t* trellis, int kin, int n, int bits, uint16_t* out) {
    if (!trellis || !out) return fail(GFR_EINVAL, "null argument");
    if (kin <= 0 || n <= 0 || kin % 16 || n % 16) return fail(GFR_EINVAL, "kin %d / n %d not multiples of 16", kin, n);
    if (bits < 2 || bits > 5) return fail(GFR_EINVAL, "bits %d outside 2..5", bits);
    hipError_t e = gfr::launch_decode_tiles(stream, trellis, kin, n, bits, out);
    if (e != hipSuccess) return hip_fail(e, "decode tiles");
    return 0;
}

// ---- prefill experts --------------------------------------------------------------------------------------------
int gfr_fast_experts_create(gfr_fast_experts** out, int hidden, int inter, int slots, int exl3_slots, int experts,
                            int max_rows) {
    if (!out) return fail(GFR_EINVAL, "null out");
    *out = nullptr;
    int rc = check_shape(hidden, inter);
    if (rc) return rc;
    if (slots <= 0 || slots > 32 || exl3_slots < 0 || exl3_slots > slots)
        return fail(GFR_EINVAL, "slots %d / exl3_slots %d", slots, exl3_slots);
    if (experts <= 0 || experts > 4096) return fail(GFR_EINVAL, "experts %d", experts);
    if (max_rows <= 0 || max_rows > (1 << 16)) return fail(GFR_EINVAL, "expert prefill scratch bound: %d", max_rows);
    gfr_fast_experts* fx = nullptr;
    hipError_t e = gfr::prefill_create(&fx, hidden, inter, slots, exl3_slots, experts, max_rows);
    if (e != hipSuccess) return hip_fail(e, "prefill scratch");
    *out = fx;
    return 0;
}

int gfr_fast_experts_run(gfr_fast_experts* fx, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                         int input_stride, const int32_t* picks, const int32_t* ids, const int32_t* count,
                         const int32_t* members, int rows, int maxm, int shared_x) {
    if (!fx) return fail(GFR_EINVAL, "null fast experts");
    const gfr::PrefillDims d = gfr::prefill_dims(fx);
    int rc = check_weights(w, d.hidden, d.inter);
    if (rc) return rc;
    if (!(rows > 0 && rows <= d.max_rows && maxm >= rows && maxm <= d.max_rows))
        return fail(GFR_EINVAL, "expert rows/member stride outside scratch: rows %d maxm %d max_rows %d", rows, maxm,
                    d.max_rows);
    if (w->experts > d.experts) return fail(GFR_EINVAL, "weights hold %d experts, engine %d", w->experts, d.experts);
    if (!input || !picks || !ids || !count || !members) return fail(GFR_EINVAL, "null input");
    if (input_stride < d.hidden) return fail(GFR_EINVAL, "input stride %d < hidden %d", input_stride, d.hidden);
    hipError_t e = gfr::prefill_run(fx, stream, w, input, input_stride, picks, ids, count, members, rows, maxm,
                                    shared_x != 0);
    if (e != hipSuccess) return hip_fail(e, "prefill run");
    return 0;
}

float* gfr_fast_experts_output(const gfr_fast_experts* fx) { return fx ? gfr::prefill_output(fx) : nullptr; }
uint16_t* gfr_fast_experts_xd(const gfr_fast_experts* fx) { return fx ? gfr::prefill_xd(fx) : nullptr; }
uint16_t* gfr_fast_experts_rotated(const gfr_fast_experts* fx, int mat) {
    return fx && (mat == 0 || mat == 1) ? gfr::prefill_rotated(fx, mat) : nullptr;
}
int gfr_fast_experts_destroy(gfr_fast_experts* fx) {
    gfr::prefill_destroy(fx);
    return 0;
}

// ---- one MoE layer ----------------------------------------------------------------------------------------------
int gfr_moe_create(gfr_moe** out, int hidden, int inter, int routed, int topk, int max_rows) {
    return gfr_moe_create_shared(out, hidden, inter, routed, topk, max_rows, 1);
}

int gfr_moe_create_shared(gfr_moe** out, int hidden, int inter, int routed, int topk, int max_rows, int shared_exl3) {
    if (!out) return fail(GFR_EINVAL, "null out");
    *out = nullptr;
    int rc = check_shape(hidden, inter);
    if (rc) return rc;
    if (routed <= 0 || routed > 1023) return fail(GFR_EINVAL, "routed experts %d outside 1..1023", routed);
    if (topk <= 0 || topk > 31 || topk > routed) return fail(GFR_EINVAL, "topk %d", topk);
    if (max_rows <= 0 || max_rows > (1 << 16)) return fail(GFR_EINVAL, "max_rows %d", max_rows);
    // decode engine for up to 64 rows; by default it takes windows of at most MOE_DECODE_ROWS rows, the prefill
    // engine (split-K MFMA for small windows) the rest: measured on MI355X (Zipf(1.1) routing), the decode engine wins
    // up to 4 rows and split-K from 6 at both benchmark shapes (hidden 2048 top-4: 49.8 / 57.9 us at 4 rows, 72.2 /
    // 63.6 at 6; hidden 5120 top-8 K = 3: 169 / 173 at 4, 256 / 204 at 6)
    constexpr int MOE_DECODE_ROWS = 4;
    const int dec_cap = 64 < max_rows ? 64 : max_rows;
    gfr_moe* m = new gfr_moe{hidden, inter, routed, topk, topk + 1, max_rows,
                             MOE_DECODE_ROWS < max_rows ? MOE_DECODE_ROWS : max_rows,
                             nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1.f,
                             shared_exl3 ? 1 : 0, nullptr, 0, nullptr, nullptr};
    const int exl3_slots = shared_exl3 ? topk + 1 : topk, experts = shared_exl3 ? routed + 1 : routed;
    m->route_bias = nullptr;   // the softmax gate until gfr_moe_set_router
    m->route_scale = 1.f;
    const size_t P = (size_t)max_rows * m->slots;
    if ((rc = alloc_zero(&m->weights, P, "moe weights")) || (rc = alloc_zero(&m->picks, P, "moe picks")) ||
        (rc = alloc_zero(&m->out, (size_t)max_rows * hidden, "moe output")) ||
        (rc = alloc_zero(&m->logits, (size_t)max_rows * routed, "moe logits")) ||
        (rc = gfr_grouping_create(&m->group_dec, routed + 1, m->slots, dec_cap)) ||
        (rc = gfr_experts_create(&m->dec, hidden, inter, m->slots, exl3_slots, dec_cap))) {
        gfr_moe_destroy(m);
        return rc;
    }
    // the reference's layout: the FP8 shared expert's engine, for gfr_moe_run_fp8 / gfr_moe_run_router_fp8
    if (!shared_exl3 && hidden % 512 == 0 &&
        ((rc = gfr_shared_fp8_create(&m->sfp8, hidden, inter, max_rows)) ||
         (rc = alloc_zero(&m->shared_out, (size_t)max_rows * hidden, "moe shared output")))) {
        gfr_moe_destroy(m);
        return rc;
    }
    if (max_rows > m->decode_rows &&
        ((rc = gfr_grouping_create(&m->group_pre, routed + 1, m->slots, max_rows)) ||
         (rc = gfr_fast_experts_create(&m->pre, hidden, inter, m->slots, exl3_slots, experts, max_rows)))) {
        gfr_moe_destroy(m);
        return rc;
    }
    *out = m;
    return 0;
}

int gfr_moe_set_decode_rows(gfr_moe* m, int decode_rows) {
    if (!m) return fail(GFR_EINVAL, "null moe");
    if (decode_rows < 0 || decode_rows > m->dec->max_rows || decode_rows > m->group_dec->max_rows)
        return fail(GFR_EINVAL, "decode_rows %d outside 0..%d", decode_rows, m->dec->max_rows);
    if (decode_rows < m->max_rows && !m->pre)
        return fail(GFR_EINVAL, "decode_rows %d leaves rows for the prefill engine, which this layer lacks",
                    decode_rows);
    m->decode_rows = decode_rows;
    return 0;
}

namespace {
int moe_run(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input, const float* logits,
            const float* shared, int shared_stride, int rows, hipEvent_t shared_ready = nullptr,
            const gfr::Fp8Shared* fp8 = nullptr) {
    if (!m) return fail(GFR_EINVAL, "null moe");
    int rc = check_weights(w, m->hidden, m->inter);
    if (rc) return rc;
    if (w->experts != m->routed + m->shared_exl3)
        return fail(GFR_EINVAL, "weights hold %d experts, layer needs %d routed%s", w->experts, m->routed,
                    m->shared_exl3 ? " + 1 shared" : "");
    if (rows <= 0 || rows > m->max_rows) return fail(GFR_EINVAL, "rows %d outside 1..%d", rows, m->max_rows);
    if (!input || !logits) return fail(GFR_EINVAL, "null input");
    if (shared && m->shared_exl3) return fail(GFR_EINVAL, "the layer's shared expert is EXL3: no shared output");
    if (shared && shared_stride < m->hidden) return fail(GFR_EINVAL, "shared stride %d < hidden %d", shared_stride,
                                                         m->hidden);
    // the combine reads the shared rows 16 bytes at a time
    if (shared && (shared_stride % 4 || reinterpret_cast<uintptr_t>(shared) % 16))
        return fail(GFR_EINVAL, "shared output: stride %d must be a multiple of 4 and the pointer 16-byte aligned",
                    shared_stride);
    if (shared_ready && !shared) return fail(GFR_EINVAL, "a shared-ready event without a shared output");
    hipError_t e;
    if (rows <= m->decode_rows) {
        gfr_grouping* g = m->group_dec;
        if (rows == 1) {
            // three launches: gate/up (+ route, rotation), down (+ gate/up epilogue), down epilogue (+ combine)
            const gfr::RouteOne r{logits, m->route_bias, m->route_scale, m->routed, m->picks, m->weights, g->ids,
                                  g->count, g->members};
            return experts_run(m->dec, stream, w, input, m->hidden, m->picks, g->ids, g->count, g->members, 1,
                               g->max_rows, m->weights, m->out, &r, shared, shared_stride, m->launches,
                               shared_ready, fp8);
        }
        // four launches: route + group, gate/up (+ rotation), down (+ gate/up epilogue), down epilogue (+ combine)
        if ((e = gfr::launch_route_group(stream, logits, rows, m->routed, m->topk, m->picks, m->weights, g->ids,
                                         g->count, g->members, g->max_rows, 0, nullptr, nullptr, nullptr, 0,
                                         m->route_bias, m->route_scale)) != hipSuccess)
            return hip_fail(e, "route + group");
        return experts_run(m->dec, stream, w, input, m->hidden, m->picks, g->ids, g->count, g->members, rows,
                           g->max_rows, m->weights, m->out, nullptr, shared, shared_stride, 0, shared_ready);
    }
    gfr_grouping* g = m->group_pre;
    bool planned = false, rotated = false;
    if ((e = gfr::launch_route_group_rot(m->pre, stream, w, input, m->hidden, logits, rows, m->routed, m->topk,
                                         m->picks, m->weights, g->ids, g->count, g->members, g->max_rows,
                                         m->route_bias, m->route_scale)) == hipSuccess) {
        // route + group + item plan and the input rotation in one launch
        planned = rotated = true;
    } else if (e != hipErrorNotSupported) {
        return hip_fail(e, "route + group + rotation");
    } else if (rows <= gfr::GROUP_SMALL_ROWS && g->experts <= 1024 &&
        gfr::route_group_lds(rows, m->slots, g->experts) <= gfr::GROUP_LDS_MAX) {
        // route + group + the prefill engine's item plan in one launch (the same router, grouping and plan as the
        // separate launches below)
        int *pu, *pi, *pp;
        gfr::prefill_plan_buffers(m->pre, &pu, &pi, &pp);
        if ((e = gfr::launch_route_group(stream, logits, rows, m->routed, m->topk, m->picks, m->weights, g->ids,
                                         g->count, g->members, g->max_rows,
                                         gfr::prefill_item_rows(m->pre, rows, w->bits), pu, pi, pp, w->experts,
                                         m->route_bias, m->route_scale)) != hipSuccess)
            return hip_fail(e, "route + group");
        planned = true;
    } else {
        if ((e = gfr::launch_route(stream, logits, rows, m->routed, m->topk, m->routed, m->picks, m->weights,
                                   m->route_bias, m->route_scale)) != hipSuccess)
            return hip_fail(e, "route");
        if (rows <= gfr::GROUP_SMALL_ROWS) {
            if ((rc = gfr_grouping_run(g, stream, m->picks, rows))) return rc;
        } else {
            // the three grouping launches, the last of which also writes the item plan and rotates the input
            if ((e = gfr::launch_group_large_rot(m->pre, stream, w, input, m->hidden, m->picks, rows, g->slots,
                                                 g->experts, g->bits, g->first, g->prefix, g->counts, g->ids,
                                                 g->count, g->members, g->max_rows)) == hipSuccess) {
                rotated = true;
            } else if (e != hipErrorNotSupported) {
                return hip_fail(e, "grouping + rotation launches");
            } else {
                int *pu, *pi, *pp;
                gfr::prefill_plan_buffers(m->pre, &pu, &pi, &pp);
                if ((e = gfr::launch_group_large(stream, m->picks, rows, g->slots, g->experts, g->bits, g->first,
                                                 g->prefix, g->counts, g->ids, g->count, g->members, g->max_rows,
                                                 gfr::prefill_item_rows(m->pre, rows, w->bits), pu, pi, pp,
                                                 w->experts)) != hipSuccess)
                    return hip_fail(e, "grouping launch");
            }
            planned = true;
        }
    }
    // windows on the split-K programs fold the combine into their down epilogue
    bool combined = false;
    if ((e = gfr::prefill_run(m->pre, stream, w, input, m->hidden, m->picks, g->ids, g->count, g->members, rows,
                              g->max_rows, false, m->weights, m->out, &combined, planned, shared, shared_stride,
                              shared_ready, rotated)) != hipSuccess)
        return hip_fail(e, "prefill run");
    if (!combined && shared_ready && (e = hipStreamWaitEvent(stream, shared_ready, 0)) != hipSuccess)
        return hip_fail(e, "wait for the shared expert");
    if (!combined &&
        (e = gfr::launch_combine(stream, gfr::prefill_output(m->pre), m->weights, rows, m->slots,
                                 m->shared_exl3 ? m->slots : m->slots - 1, m->hidden, shared, shared_stride,
                                 m->out)) != hipSuccess)
        return hip_fail(e, "combine");
    return 0;
}
}  // namespace

int gfr_moe_run(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                const float* logits, int rows) {
    return moe_run(m, stream, w, input, logits, nullptr, 0, rows);
}

// ---- the bs = 1 layer without allocation ----------------------------------------------------------------------
// Every scratch buffer of gfr_moe_token_static lives in this fixed device array (one per GPU, held until the process
// ends). Host code uses the per-device address from hipGetSymbolAddress, never the array's name.
}  // extern "C"
namespace {
constexpr size_t STATIC_SCRATCH_BYTES = (size_t)8 << 20;
static __device__ __align__(256) unsigned char scratch[STATIC_SCRATCH_BYTES];
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mutex;
void* g_scratch[MAX_DEVICES];

// this device's address of `scratch` (looked up once per device, with that device current)
int scratch_ptr(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "static scratch: current device");
    if (dev < 0 || dev >= MAX_DEVICES) return fail(GFR_EUNSUPPORTED, "static scratch: device %d", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return hip_fail(e != hipSuccess ? e : hipErrorInvalidSymbol, "static scratch address");
        g_scratch[dev] = p;
    }
    *out = g_scratch[dev];
    return 0;
}

// carve 256-byte aligned pieces off the array
struct Carver {
    unsigned char* base;
    size_t off;
    template <typename T>
    T* take(size_t count) {
        T* p = reinterpret_cast<T*>(base + off);
        off += (count * sizeof(T) + 255) & ~(size_t)255;
        return p;
    }
};
}  // namespace
extern "C" {

int gfr_moe_token_static(hipStream_t stream, const gfr_exl3_experts* w, int routed, int topk, const uint16_t* input,
                         const float* logits, float* out, int32_t* picks, float* weights) {
    if (!w) return fail(GFR_EINVAL, "null weights");
    int rc = check_shape(w->hidden, w->inter);
    if (rc) return rc;
    rc = check_weights(w, w->hidden, w->inter);
    if (rc) return rc;
    if (routed <= 0 || routed > 1023 || topk <= 0 || topk > 31 || topk > routed)
        return fail(GFR_EINVAL, "routed %d / topk %d", routed, topk);
    if (w->experts != routed + 1)
        return fail(GFR_EINVAL, "weights hold %d experts, layer needs %d routed + 1 shared", w->experts, routed);
    if (!input || !logits || !out) return fail(GFR_EINVAL, "null input, logits or output");
    const int slots = topk + 1, D = w->hidden, N = w->inter;
    // the layout, sized first on a null base, then placed on this device's array
    int32_t *pk, *ids, *count, *members;
    float* wt;
    gfr_experts ex{D, N, slots, slots, 1, nullptr, nullptr, nullptr, nullptr};
    auto carve = [&](Carver& c) {
        pk = c.take<int32_t>(slots);
        wt = c.take<float>(slots);
        ids = c.take<int32_t>(slots);
        count = c.take<int32_t>(1);
        members = c.take<int32_t>(slots);
        ex.zgu = c.take<float>((size_t)2 * gfr::gemv_gateup_splits(D) * slots * N);
        ex.xd = c.take<uint16_t>((size_t)slots * N);
        ex.zd = c.take<float>((size_t)gfr::gemv_down_splits(N) * slots * D);
        ex.y = c.take<float>((size_t)slots * D);
    };
    Carver size{nullptr, 0};
    carve(size);
    if (size.off > STATIC_SCRATCH_BYTES)
        return fail(GFR_EINVAL, "layer hidden %d inter %d top-%d needs %zu bytes of scratch, the static array holds %zu",
                    D, N, topk, size.off, STATIC_SCRATCH_BYTES);
    void* base = nullptr;
    if ((rc = scratch_ptr(&base))) return rc;
    Carver c{static_cast<unsigned char*>(base), 0};
    carve(c);
    const gfr::RouteOne r{logits, nullptr, 1.f, routed, pk, wt, ids, count, members};
    if ((rc = experts_run(&ex, stream, w, input, D, pk, ids, count, members, 1, 1, wt, out, &r))) return rc;
    hipError_t e;
    if (picks && (e = hipMemcpyAsync(picks, pk, slots * 4, hipMemcpyDeviceToDevice, stream)) != hipSuccess)
        return hip_fail(e, "picks copy");
    if (weights && (e = hipMemcpyAsync(weights, wt, slots * 4, hipMemcpyDeviceToDevice, stream)) != hipSuccess)
        return hip_fail(e, "weights copy");
    return 0;
}

int gfr_moe_run_shared(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                       const float* logits, const float* shared, int shared_stride, int rows) {
    if (!shared) return fail(GFR_EINVAL, "null shared output");
    return moe_run(m, stream, w, input, logits, shared, shared_stride, rows);
}

int gfr_moe_run_shared_branch(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                              const float* logits, const float* shared, int shared_stride, int rows,
                              hipEvent_t shared_ready) {
    if (!shared || !shared_ready) return fail(GFR_EINVAL, "null shared output or event");
    return moe_run(m, stream, w, input, logits, shared, shared_stride, rows, shared_ready);
}

int gfr_moe_run_router(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                       const uint16_t* router_weight, const float* shared, int shared_stride, int rows) {
    if (!m) return fail(GFR_EINVAL, "null moe");
    if (!input || !router_weight) return fail(GFR_EINVAL, "null input or router weight");
    if (rows <= 0 || rows > m->max_rows) return fail(GFR_EINVAL, "rows %d outside 1..%d", rows, m->max_rows);
    int rc = gfr_router_logits(stream, input, m->hidden, router_weight, m->hidden, m->routed, rows, m->logits);
    if (rc) return rc;
    return moe_run(m, stream, w, input, m->logits, shared, shared_stride, rows);
}

// ---- the FP8 shared expert --------------------------------------------------------------------------------------
namespace {
// windows of up to this many rows run the slice arithmetic of the reference's decode / verify path (fmm, moe.rs and
// window_gemm.rs, MAX_ROWS 16 in kda_window.rs); larger ones its prefill form when the bf16 copies are given
constexpr int FP8_SLICE_ROWS = 16;
bool al16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
int check_fp8_weights(const gfr_fp8_shared_weights* w, int hidden, int inter) {
    if (!w) return fail(GFR_EINVAL, "null FP8 shared weights");
    if (w->hidden != hidden || w->inter != inter)
        return fail(GFR_EINVAL, "FP8 shared weights %dx%d, engine %dx%d", w->hidden, w->inter, hidden, inter);
    if (!w->gu || !w->gu_scale || !w->down || !w->down_scale) return fail(GFR_EINVAL, "null FP8 shared tensor");
    if (!al16(w->gu) || !al16(w->gu_scale) || !al16(w->down) || !al16(w->down_scale))
        return fail(GFR_EINVAL, "FP8 shared tensors must be 16-byte aligned");
    return 0;
}
int shared_fp8_run(gfr_shared_fp8* sh, hipStream_t stream, const gfr_fp8_shared_weights* w, const uint16_t* input,
                   int input_stride, int rows, float* out, int out_stride) {
    if (!sh) return fail(GFR_EINVAL, "null FP8 shared engine");
    int rc = check_fp8_weights(w, sh->hidden, sh->inter);
    if (rc) return rc;
    if (rows <= 0 || rows > sh->max_rows) return fail(GFR_EINVAL, "rows %d outside 1..%d", rows, sh->max_rows);
    if (!input || !out) return fail(GFR_EINVAL, "null input or output");
    // rows are read 16 bytes at a time and written 16 bytes at a time
    if (input_stride < sh->hidden || input_stride % 8 || !al16(input))
        return fail(GFR_EINVAL, "input stride %d: at least hidden %d, a multiple of 8, the pointer 16-byte aligned",
                    input_stride, sh->hidden);
    if (out_stride < sh->hidden || out_stride % 4 || !al16(out))
        return fail(GFR_EINVAL, "output stride %d: at least hidden %d, a multiple of 4, the pointer 16-byte aligned",
                    out_stride, sh->hidden);
    hipError_t e;
    if (rows > FP8_SLICE_ROWS && w->gu_bf16 && w->down_bf16 && sh->blas) {
        if (!al16(w->gu_bf16) || !al16(w->down_bf16))
            return fail(GFR_EINVAL, "FP8 shared bf16 weight copies must be 16-byte aligned");
        e = gfr::launch_shared_fp8_prefill(sh->blas, stream, w->gu_bf16, w->down_bf16, input, input_stride, rows,
                                           sh->hidden, sh->inter, sh->gu, sh->act, out, out_stride);
    } else {
        e = gfr::launch_shared_fp8(stream, w->gu, w->gu_scale, w->down, w->down_scale, input, input_stride, rows,
                                   sh->hidden, sh->inter, sh->gu, sh->act, out, out_stride);
    }
    if (e != hipSuccess) return hip_fail(e, "FP8 shared expert");
    return 0;
}
int moe_fp8_ready(gfr_moe* m, const gfr_fp8_shared_weights* sw) {
    if (!m) return fail(GFR_EINVAL, "null moe");
    if (m->shared_exl3 || !m->sfp8)
        return fail(GFR_EINVAL, "the layer has no FP8 shared expert (made with shared_exl3 = 1, or hidden %d is not "
                    "a multiple of 512)", m->hidden);
    return check_fp8_weights(sw, m->hidden, m->inter);
}
}  // namespace

int gfr_shared_fp8_create(gfr_shared_fp8** out, int hidden, int inter, int max_rows) {
    if (!out) return fail(GFR_EINVAL, "null out");
    *out = nullptr;
    if (hidden <= 0 || hidden % 512 || hidden > (1 << 20) || inter <= 0 || inter % 64 || inter > (1 << 20))
        return fail(GFR_EINVAL, "FP8 shared expert: hidden %d a multiple of 512, inter %d of 64", hidden, inter);
    if (max_rows <= 0 || max_rows > (1 << 16)) return fail(GFR_EINVAL, "max_rows %d", max_rows);
    gfr_shared_fp8* sh = new gfr_shared_fp8{hidden, inter, max_rows, nullptr, nullptr, nullptr, nullptr};
    int rc;
    if ((rc = alloc_zero(&sh->gu, (size_t)max_rows * 2 * inter, "FP8 shared gu")) ||
        (rc = alloc_zero(&sh->act, (size_t)max_rows * inter, "FP8 shared activation"))) {
        gfr_shared_fp8_destroy(sh);
        return rc;
    }
    if (max_rows > FP8_SLICE_ROWS) {
        // windows past the verify size may take the prefill form (library GEMMs on the bf16 weight copies)
        constexpr size_t WS = (size_t)64 << 20;
        unsigned char* ws = nullptr;
        if ((rc = alloc_zero(&ws, WS, "FP8 shared GEMM workspace"))) {
            gfr_shared_fp8_destroy(sh);
            return rc;
        }
        sh->blas_ws = ws;
        if (rocblas_create_handle(&sh->blas) != rocblas_status_success ||
            rocblas_set_workspace(sh->blas, sh->blas_ws, WS) != rocblas_status_success) {
            gfr_shared_fp8_destroy(sh);
            return fail(GFR_ENOMEM, "FP8 shared expert: rocBLAS handle");
        }
    }
    *out = sh;
    return 0;
}

int gfr_fp8_prepare_bf16(hipStream_t stream, const gfr_fp8_shared_weights* w, uint16_t* gu_bf16,
                         uint16_t* down_bf16) {
    if (!w || !w->gu || !w->gu_scale || !w->down || !w->down_scale || !gu_bf16 || !down_bf16)
        return fail(GFR_EINVAL, "null FP8 shared tensor or output");
    if (w->hidden <= 0 || w->hidden % 16 || w->inter <= 0 || w->inter % 16)
        return fail(GFR_EINVAL, "FP8 shared expert: hidden %d and inter %d multiples of 16", w->hidden, w->inter);
    if (!al16(w->gu) || !al16(w->down) || !al16(gu_bf16) || !al16(down_bf16))
        return fail(GFR_EINVAL, "FP8 weights and their bf16 copies must be 16-byte aligned");
    hipError_t e;
    if ((e = gfr::launch_fp8_b16_copy(stream, w->gu, w->gu_scale, gu_bf16, 2 * w->inter, w->hidden)) != hipSuccess ||
        (e = gfr::launch_fp8_b16_copy(stream, w->down, w->down_scale, down_bf16, w->hidden, w->inter)) != hipSuccess)
        return hip_fail(e, "FP8 -> bf16 weight copies");
    return 0;
}

int gfr_shared_fp8_run(gfr_shared_fp8* sh, hipStream_t stream, const gfr_fp8_shared_weights* w,
                       const uint16_t* input, int input_stride, int rows, float* out, int out_stride) {
    return shared_fp8_run(sh, stream, w, input, input_stride, rows, out, out_stride);
}

uint16_t* gfr_shared_fp8_gu(const gfr_shared_fp8* sh) { return sh ? sh->gu : nullptr; }
uint16_t* gfr_shared_fp8_act(const gfr_shared_fp8* sh) { return sh ? sh->act : nullptr; }

int gfr_shared_fp8_destroy(gfr_shared_fp8* sh) {
    if (!sh) return 0;
    if (sh->blas) rocblas_destroy_handle(sh->blas);
    free_all({sh->gu, sh->act, sh->blas_ws});
    delete sh;
    return 0;
}

namespace {
// The layer with its FP8 shared expert. A one-token window whose launches have the shared slot's workgroups (the
// grid's last unit exists: the weights hold at least `slots` experts) runs the shared expert inside the gate/up and
// down launches (three launches in all); other windows run its two launches first.
int moe_run_fp8(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                const float* logits, const gfr_fp8_shared_weights* sw, int rows) {
    if (rows <= 0 || rows > m->max_rows) return fail(GFR_EINVAL, "rows %d outside 1..%d", rows, m->max_rows);
    if (!w || !input) return fail(GFR_EINVAL, "null weights or input");
    if (!al16(input)) return fail(GFR_EINVAL, "input rows must be 16-byte aligned");
    const bool fused = rows == 1 && rows <= m->decode_rows && w->experts >= m->slots &&
                       gfr::gemv_gateup_splits(m->hidden) <= 16;
    if (!fused) {
        int rc = shared_fp8_run(m->sfp8, stream, sw, input, m->hidden, rows, m->shared_out, m->hidden);
        if (rc) return rc;
        return moe_run(m, stream, w, input, logits, m->shared_out, m->hidden, rows);
    }
    const gfr::Fp8Shared job{sw->gu, sw->gu_scale, sw->down, sw->down_scale, m->sfp8->gu, m->sfp8->act,
                             m->shared_out, m->hidden, m->inter};
    return moe_run(m, stream, w, input, logits, m->shared_out, m->hidden, rows, nullptr, &job);
}
}  // namespace

int gfr_moe_run_fp8(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                    const float* logits, const gfr_fp8_shared_weights* sw, int rows) {
    int rc = moe_fp8_ready(m, sw);
    if (rc) return rc;
    return moe_run_fp8(m, stream, w, input, logits, sw, rows);
}

int gfr_moe_run_router_fp8(gfr_moe* m, hipStream_t stream, const gfr_exl3_experts* w, const uint16_t* input,
                           const uint16_t* router_weight, const gfr_fp8_shared_weights* sw, int rows) {
    int rc = moe_fp8_ready(m, sw);
    if (rc) return rc;
    if (!input || !router_weight) return fail(GFR_EINVAL, "null input or router weight");
    if (rows <= 0 || rows > m->max_rows) return fail(GFR_EINVAL, "rows %d outside 1..%d", rows, m->max_rows);
    if ((rc = gfr_router_logits(stream, input, m->hidden, router_weight, m->hidden, m->routed, rows, m->logits)))
        return rc;
    return moe_run_fp8(m, stream, w, input, m->logits, sw, rows);
}

float* gfr_moe_shared_output(const gfr_moe* m) { return m ? m->shared_out : nullptr; }

int gfr_router_logits(hipStream_t stream, const uint16_t* input, int input_stride, const uint16_t* router_weight,
                      int hidden, int routed, int rows, float* logits) {
    if (!input || !router_weight || !logits) return fail(GFR_EINVAL, "null argument");
    if (hidden <= 0 || hidden % 8 || hidden > gfr::router_logits_max_hidden())
        return fail(GFR_EINVAL, "router hidden %d: a positive multiple of 8 up to %d", hidden,
                    gfr::router_logits_max_hidden());
    if (routed <= 0 || rows <= 0 || input_stride < hidden)
        return fail(GFR_EINVAL, "routed %d rows %d stride %d", routed, rows, input_stride);
    // the logits kernel reads input and weight rows 16 bytes at a time
    if (input_stride % 8 || reinterpret_cast<uintptr_t>(input) % 16 || reinterpret_cast<uintptr_t>(router_weight) % 16)
        return fail(GFR_EINVAL, "router input stride %d must be a multiple of 8 and both pointers 16-byte aligned",
                    input_stride);
    hipError_t e = gfr::launch_router_logits(stream, input, input_stride, router_weight, hidden, routed, rows, logits);
    if (e != hipSuccess) return hip_fail(e, "router logits");
    return 0;
}

int gfr_moe_set_launches(gfr_moe* m, int launches) {
    if (!m) return fail(GFR_EINVAL, "null moe");
    if (launches < 0 || launches > 3) return fail(GFR_EINVAL, "launches %d outside 0..3", launches);
    m->launches = launches == 3 ? 0 : launches;
    return 0;
}

int gfr_moe_set_router(gfr_moe* m, const float* bias, float scale) {
    if (!m) return fail(GFR_EINVAL, "null moe");
    if (bias && !(scale > 0.f)) return fail(GFR_EINVAL, "router scale %g must be positive", (double)scale);
    m->route_bias = bias;
    m->route_scale = bias ? scale : 1.f;
    return 0;
}

float* gfr_moe_output(const gfr_moe* m) { return m ? m->out : nullptr; }
int32_t* gfr_moe_picks(const gfr_moe* m) { return m ? m->picks : nullptr; }
float* gfr_moe_weights(const gfr_moe* m) { return m ? m->weights : nullptr; }
uint16_t* gfr_moe_rotated(const gfr_moe* m, int mat) {
    return m && (mat == 0 || mat == 1) ? gfr::prefill_rotated(m->pre, mat) : nullptr;
}

int gfr_moe_destroy(gfr_moe* m) {
    if (!m) return 0;
    gfr_grouping_destroy(m->group_dec);
    gfr_grouping_destroy(m->group_pre);
    gfr_experts_destroy(m->dec);
    gfr_fast_experts_destroy(m->pre);
    gfr_shared_fp8_destroy(m->sfp8);
    free_all({m->weights, m->picks, m->out, m->logits, m->shared_out});
    delete m;
    return 0;
}

}  // extern "C"
