// vo_gemm.cpp -- Backend::matmul (crates/engine/src/backend/mod.rs:98,
// cpu/mod.rs:199-229) on hipBLASLt: out[rows, N] = x[rows, K] . W^T with W
// [N, K] bf16, the reference's weight layout, fp32 accumulation.
//
// hipBLASLt is column-major.  A row-major [N, K] weight is, read column-major,
// a K x N matrix with leading dimension K; the row-major x [rows, K] is a
// K x rows matrix.  So out^T (column-major N x rows, ld N -- the row-major
// [rows, N] output) = op(A) . B with A = W (K x N, transposed), B = x (K x
// rows, not transposed): the "TN" GEMM.  With accumulate, beta = 1 and C is
// the output itself: the model's residual add folded into the epilogue.
//
// The library is opened with dlopen when a vo_gemm is created: in a process
// that already has hipBLASLt mapped (PyTorch-ROCm loads its bundled copy with
// the same SONAME), that copy -- built for the HIP runtime the process uses
// -- is the one bound; otherwise libhipblaslt.so.1 from the loader path.
// Nothing else in the library depends on it.
//
// Algorithm choice, once per (rows, N, K, out type, accumulate), cached with
// its descriptors: hipBLASLt's first heuristic choice, or with VO_GEMM_TUNE=1
// the fastest of its candidates timed on the first call's operands (on the
// Llama-3-8B step shapes the two measured the same).
// Later calls allocate nothing (the workspace is allocated at creation) and
// may be captured in a HIP graph; the first call of a shape may not.  Shapes whose rows are not whole 16-byte words go to a generic
// kernel (kernels/layer_ops.hip).
#include <dlfcn.h>
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <type_traits>
#include <map>
#include <mutex>
#include <string>
#include <tuple>

#include "vo_backend.hpp"

using namespace vo;

namespace {

struct LtApi {
    void *handle = nullptr;
    decltype(&hipblasLtCreate) create = nullptr;
    decltype(&hipblasLtDestroy) destroy = nullptr;
    decltype(&hipblasLtMatmulDescCreate) desc_create = nullptr;
    decltype(&hipblasLtMatmulDescDestroy) desc_destroy = nullptr;
    decltype(&hipblasLtMatmulDescSetAttribute) desc_set = nullptr;
    decltype(&hipblasLtMatrixLayoutCreate) layout_create = nullptr;
    decltype(&hipblasLtMatrixLayoutDestroy) layout_destroy = nullptr;
    decltype(&hipblasLtMatmulPreferenceCreate) pref_create = nullptr;
    decltype(&hipblasLtMatmulPreferenceDestroy) pref_destroy = nullptr;
    decltype(&hipblasLtMatmulPreferenceSetAttribute) pref_set = nullptr;
    decltype(&hipblasLtMatmulAlgoGetHeuristic) heuristic = nullptr;
    decltype(&hipblasLtMatmul) matmul = nullptr;
    std::string error;
};

// Opens hipBLASLt once per process; `error` says why when it cannot.
const LtApi &lt_api() {
    static LtApi api;
    static std::once_flag once;
    std::call_once(once, [] {
        void *h = dlopen("libhipblaslt.so.1", RTLD_NOW | RTLD_NOLOAD);
        if (!h) h = dlopen("libhipblaslt.so.1", RTLD_NOW);
        if (!h) h = dlopen("/opt/rocm/lib/libhipblaslt.so.1", RTLD_NOW);
        if (!h) {
            const char *e = dlerror();
            api.error = std::string("cannot load libhipblaslt.so.1: ") + (e ? e : "unknown");
            return;
        }
        bool ok = true;
        auto sym = [&](auto &fn, const char *name) {
            fn = reinterpret_cast<std::remove_reference_t<decltype(fn)>>(dlsym(h, name));
            if (!fn) {
                ok = false;
                api.error = std::string("libhipblaslt.so.1 lacks ") + name;
            }
        };
        sym(api.create, "hipblasLtCreate");
        sym(api.destroy, "hipblasLtDestroy");
        sym(api.desc_create, "hipblasLtMatmulDescCreate");
        sym(api.desc_destroy, "hipblasLtMatmulDescDestroy");
        sym(api.desc_set, "hipblasLtMatmulDescSetAttribute");
        sym(api.layout_create, "hipblasLtMatrixLayoutCreate");
        sym(api.layout_destroy, "hipblasLtMatrixLayoutDestroy");
        sym(api.pref_create, "hipblasLtMatmulPreferenceCreate");
        sym(api.pref_destroy, "hipblasLtMatmulPreferenceDestroy");
        sym(api.pref_set, "hipblasLtMatmulPreferenceSetAttribute");
        sym(api.heuristic, "hipblasLtMatmulAlgoGetHeuristic");
        sym(api.matmul, "hipblasLtMatmul");
        if (ok) api.handle = h;
    });
    return api;
}

// One cached problem: descriptors plus the chosen algorithm.
struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t workspace = 0;
};

using PlanKey = std::tuple<uint64_t, uint64_t, uint64_t, int32_t, int32_t>;

}  // namespace

constexpr int kTuneCandidates = 16;  // heuristic candidates timed per shape
constexpr int kTuneRepeats = 5;      // timed runs per candidate

struct vo_gemm {
    int device = 0;
    bool tune = false;  // time the heuristic's candidates per shape (VO_GEMM_TUNE=1: on)
    hipblasLtHandle_t lt = nullptr;
    void *workspace = nullptr;
    uint64_t workspace_bytes = 0;
    std::map<PlanKey, Plan> plans;
    std::mutex mu;
};

namespace {

vo_status lt_fail(const char *op, const char *what, hipblasStatus_t st) {
    return fail_device(op, static_cast<int>(st), (std::string(what) + " failed").c_str());
}

void destroy_plan(const LtApi &api, Plan &p) {
    if (p.a) api.layout_destroy(p.a);
    if (p.b) api.layout_destroy(p.b);
    if (p.c) api.layout_destroy(p.c);
    if (p.desc) api.desc_destroy(p.desc);
    p = Plan{};
}

// Times the heuristic's candidates on the call's own operands (beta = 0,
// into a scratch output, so an accumulating call's output is untouched) and
// keeps the fastest.  Runs once per shape, at its first call: it allocates
// and waits, so that call must not be under stream capture.  Candidates that
// fail to run are skipped; if every timing fails the heuristic's first
// choice stays.
void tune_plan(vo_gemm *g, const LtApi &api, const void *x, const void *w, uint64_t rows,
               uint64_t n, int32_t out_dtype, const hipblasLtMatmulHeuristicResult_t *cand,
               int count, hipStream_t stream, Plan &p) {
    void *scratch = nullptr;
    const uint64_t bytes = rows * n * (out_dtype == VO_DTYPE_F32 ? 4 : 2);
    hipEvent_t t0 = nullptr, t1 = nullptr;
    if (hipMalloc(&scratch, bytes) != hipSuccess) return;
    if (hipEventCreate(&t0) != hipSuccess || hipEventCreate(&t1) != hipSuccess) {
        if (t0) (void)hipEventDestroy(t0);
        (void)hipFree(scratch);
        return;
    }
    const float alpha = 1.0f, beta = 0.0f;
    float best = 0.0f;
    int best_i = -1;
    for (int i = 0; i < count; ++i) {
        if (cand[i].state != HIPBLAS_STATUS_SUCCESS || cand[i].workspaceSize > g->workspace_bytes)
            continue;
        auto run = [&]() {
            return api.matmul(g->lt, p.desc, &alpha, w, p.a, x, p.b, &beta, scratch, p.c, scratch,
                              p.c, &cand[i].algo, cand[i].workspaceSize ? g->workspace : nullptr,
                              cand[i].workspaceSize, stream);
        };
        if (run() != HIPBLAS_STATUS_SUCCESS) continue;  // warm-up
        bool ok = hipEventRecord(t0, stream) == hipSuccess;
        for (int r = 0; ok && r < kTuneRepeats; ++r) ok = run() == HIPBLAS_STATUS_SUCCESS;
        ok = ok && hipEventRecord(t1, stream) == hipSuccess && hipEventSynchronize(t1) == hipSuccess;
        float ms = 0.0f;
        if (!ok || hipEventElapsedTime(&ms, t0, t1) != hipSuccess) continue;
        if (best_i < 0 || ms < best) {
            best = ms;
            best_i = i;
        }
    }
    (void)hipStreamSynchronize(stream);
    (void)hipEventDestroy(t0);
    (void)hipEventDestroy(t1);
    (void)hipFree(scratch);
    if (best_i >= 0) {
        p.algo = cand[best_i].algo;
        p.workspace = cand[best_i].workspaceSize;
    }
}

// Builds the descriptors of one problem and asks the heuristic for its best
// algorithms that fit the workspace; with tuning on, the fastest of them on
// this call's operands is kept.
vo_status make_plan(vo_gemm *g, const LtApi &api, uint64_t rows, uint64_t n, uint64_t k,
                    int32_t out_dtype, const void *x, const void *w, hipStream_t stream,
                    Plan &p) {
    const char *op = "matmul";
    const hipDataType out_t = out_dtype == VO_DTYPE_F32 ? HIP_R_32F : HIP_R_16BF;
    hipblasStatus_t st = api.desc_create(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F);
    if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(op, "hipblasLtMatmulDescCreate", st);
    const int32_t trans_a = HIPBLAS_OP_T, trans_b = HIPBLAS_OP_N;
    st = api.desc_set(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &trans_a, sizeof(trans_a));
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = api.desc_set(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &trans_b, sizeof(trans_b));
    if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(op, "hipblasLtMatmulDescSetAttribute", st);
    st = api.layout_create(&p.a, HIP_R_16BF, k, n, static_cast<int64_t>(k));
    if (st == HIPBLAS_STATUS_SUCCESS) st = api.layout_create(&p.b, HIP_R_16BF, k, rows, static_cast<int64_t>(k));
    if (st == HIPBLAS_STATUS_SUCCESS) st = api.layout_create(&p.c, out_t, n, rows, static_cast<int64_t>(n));
    if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(op, "hipblasLtMatrixLayoutCreate", st);
    hipblasLtMatmulPreference_t pref = nullptr;
    st = api.pref_create(&pref);
    if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(op, "hipblasLtMatmulPreferenceCreate", st);
    const uint64_t ws = g->workspace_bytes;
    st = api.pref_set(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
    hipblasLtMatmulHeuristicResult_t result[kTuneCandidates];
    int returned = 0;
    const int want = g->tune ? kTuneCandidates : 1;
    if (st == HIPBLAS_STATUS_SUCCESS)
        st = api.heuristic(g->lt, p.desc, p.a, p.b, p.c, p.c, pref, want, result, &returned);
    api.pref_destroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(op, "hipblasLtMatmulAlgoGetHeuristic", st);
    if (returned < 1)
        return fail_unsupported(op, "hipBLASLt has no algorithm for [" + std::to_string(rows) + ", " +
                                        std::to_string(k) + "] x [" + std::to_string(n) + ", " +
                                        std::to_string(k) + "]^T");
    p.algo = result[0].algo;
    p.workspace = result[0].workspaceSize;
    if (returned > 1) tune_plan(g, api, x, w, rows, n, out_dtype, result, returned, stream, p);
    return VO_OK;
}

}  // namespace

extern "C" int32_t vo_gemm_create(int32_t device, uint64_t workspace_bytes, vo_gemm **out) {
    const char *op = "matmul";
    if (!out) return fail_argument(op, "null output");
    *out = nullptr;
    const LtApi &api = lt_api();
    if (!api.handle) return fail_unsupported(op, api.error);
    DeviceGuard guard(device);
    if (!guard.ok()) return fail_device(op, hipErrorInvalidDevice, "hipSetDevice");
    vo_gemm *g = new (std::nothrow) vo_gemm();
    if (!g) return fail_argument(op, "out of host memory");
    g->device = device;
    g->workspace_bytes = workspace_bytes;
    g->tune = env_int("VO_GEMM_TUNE", 0) != 0;
    hipblasStatus_t st = api.create(&g->lt);
    if (st != HIPBLAS_STATUS_SUCCESS) {
        delete g;
        return lt_fail(op, "hipblasLtCreate", st);
    }
    if (workspace_bytes) {
        hipError_t err = hipMalloc(&g->workspace, workspace_bytes);
        if (err != hipSuccess) {
            api.destroy(g->lt);
            delete g;
            return fail_device(op, err, hipGetErrorString(err));
        }
    }
    *out = g;
    clear_error();
    return VO_OK;
}

extern "C" void vo_gemm_destroy(vo_gemm *g) {
    if (!g) return;
    const LtApi &api = lt_api();
    DeviceGuard guard(g->device);
    for (auto &kv : g->plans) destroy_plan(api, kv.second);
    if (g->lt) api.destroy(g->lt);
    if (g->workspace) (void)hipFree(g->workspace);
    delete g;
}

extern "C" int32_t vo_matmul(vo_gemm *g, const void *x, uint64_t rows, uint64_t x_cols,
                             const void *weight, uint64_t out_features, uint64_t in_features,
                             void *out, int32_t out_dtype, int32_t accumulate, void *stream) {
    const char *op = "matmul";
    if (!g) return fail_argument(op, "null gemm");
    // arena/ops.rs:68-74
    if (in_features != x_cols)
        return fail_shape(op, "x [" + std::to_string(rows) + ", " + std::to_string(x_cols) +
                                  "], weight [" + std::to_string(out_features) + ", " +
                                  std::to_string(in_features) + "]");
    if (out_dtype != VO_DTYPE_BF16 && out_dtype != VO_DTYPE_F32)
        return fail_argument(op, "out_dtype must be VO_DTYPE_BF16 or VO_DTYPE_F32");
    if (accumulate != 0 && accumulate != 1) return fail_argument(op, "accumulate must be 0 or 1");
    if (rows == 0 || out_features == 0) {
        clear_error();
        return VO_OK;
    }
    if (!x || !weight || !out) return fail_argument(op, "null x, weight or output");
    if (rows > 0x7fffffffull || out_features > 0x7fffffffull || in_features > 0x7fffffffull)
        return fail_capacity("matmul dimension", std::max({rows, out_features, in_features}),
                             0x7fffffffull);
    const uint64_t ob = rows * out_features * (out_dtype == VO_DTYPE_F32 ? 4 : 2);
    if (overlaps(out, ob, x, rows * x_cols * 2) || overlaps(out, ob, weight, out_features * in_features * 2))
        return fail_shape(op, "output overlaps an input");
    DeviceGuard guard(g->device);
    // hipBLASLt takes rows of whole 16-byte words; other shapes (the
    // reference's tiny test model: vocab 37) run on the generic kernel.
    const bool lt_shape = in_features % 8 == 0 && out_features % 8 == 0 && aligned16(x) &&
                          aligned16(weight) && aligned16(out);
    if (!lt_shape)
        return device_status(op, kernels::launch_matmul_generic(
                                     static_cast<const uint16_t *>(x),
                                     static_cast<const uint16_t *>(weight),
                                     static_cast<uint32_t>(rows), static_cast<uint32_t>(out_features),
                                     static_cast<uint32_t>(in_features), out,
                                     out_dtype == VO_DTYPE_F32, accumulate != 0,
                                     static_cast<hipStream_t>(stream)));
    // Decode-sized batches: the weight-streaming kernel (VO_SKINNY_GEMM=0: off).
    static const bool skinny_on = env_int("VO_SKINNY_GEMM", 1) != 0;
    if (skinny_on && kernels::skinny_gemm_supported(rows, out_features, in_features))
        return device_status(op, kernels::launch_skinny_gemm(
                                     static_cast<const uint16_t *>(x),
                                     static_cast<const uint16_t *>(weight),
                                     static_cast<uint32_t>(rows), static_cast<uint32_t>(out_features),
                                     static_cast<uint32_t>(in_features), out,
                                     out_dtype == VO_DTYPE_F32, accumulate != 0,
                                     static_cast<hipStream_t>(stream)));
    const LtApi &api = lt_api();
    Plan *plan;
    {
        std::lock_guard<std::mutex> lock(g->mu);
        const PlanKey key{rows, out_features, in_features, out_dtype, accumulate};
        auto it = g->plans.find(key);
        if (it == g->plans.end()) {
            Plan p;
            if (vo_status rc = make_plan(g, api, rows, out_features, in_features, out_dtype, x, weight,
                                          static_cast<hipStream_t>(stream), p)) {
                destroy_plan(api, p);
                return rc;
            }
            it = g->plans.emplace(key, p).first;
        }
        plan = &it->second;
    }
    const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
    kernels::KernelTimer timer("matmul", static_cast<hipStream_t>(stream));
    const hipblasStatus_t st =
        api.matmul(g->lt, plan->desc, &alpha, weight, plan->a, x, plan->b, &beta, out, plan->c, out,
                   plan->c, &plan->algo, plan->workspace ? g->workspace : nullptr, plan->workspace,
                   static_cast<hipStream_t>(stream));
    if (st != HIPBLAS_STATUS_SUCCESS) return lt_fail(op, "hipblasLtMatmul", st);
    clear_error();
    return VO_OK;
}
