/* Projection GEMMs through hipBLASLt (the role cuBLAS GemmEx plays in the
 * reference, src/kernels/elementwise.cu:56-75).
 *
 * Y[N, M] = X[N, K] . W[M, K]^T, bf16 inputs, fp32 accumulation, bf16 or fp32
 * output, all row-major. In hipBLASLt's column-major terms this is
 * D(M x N) = op_T(A = W seen as K x M) . B (= X seen as K x N).
 * Descriptors and the heuristic's algorithm are cached per (N, M, K, out). */
#include "kernels.h"
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <stdio.h>
#include <stdlib.h>

#include <map>
#include <mutex>
#include <tuple>
#include <vector>

struct GemmPlan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo;
    size_t ws = 0;
};

struct cujev_gemm {
    hipblasLtHandle_t handle = nullptr;
    void *workspace = nullptr;
    size_t ws_bytes = 0;
    std::map<std::tuple<int, int, int, int>, GemmPlan> plans;
    /* tuned algorithms: (M, K, f32out) -> {N: hipBLASLt solution index} */
    std::map<std::tuple<int, int, int>, std::map<int, int>> table;
    std::map<int, std::vector<hipblasLtMatmulHeuristicResult_t>> all_algos; /* by f32out */
    std::mutex mu;
};

static void destroy_plan(GemmPlan &p) {
    if (p.desc)
        hipblasLtMatmulDescDestroy(p.desc);
    if (p.a)
        hipblasLtMatrixLayoutDestroy(p.a);
    if (p.b)
        hipblasLtMatrixLayoutDestroy(p.b);
    if (p.c)
        hipblasLtMatrixLayoutDestroy(p.c);
}

extern "C" int cujev_gemm_create(cujev_gemm **out, void *workspace, size_t ws_bytes) {
    cujev_gemm *g = new (std::nothrow) cujev_gemm();
    if (!g)
        return -1;
    if (hipblasLtCreate(&g->handle) != HIPBLAS_STATUS_SUCCESS) {
        delete g;
        return -1;
    }
    g->workspace = workspace;
    g->ws_bytes = ws_bytes;
    *out = g;
    return 0;
}

extern "C" void cujev_gemm_destroy(cujev_gemm *g) {
    if (!g)
        return;
    for (auto &kv : g->plans)
        destroy_plan(kv.second);
    if (g->handle)
        hipblasLtDestroy(g->handle);
    delete g;
}

/* By default a shape keeps the heuristic's first algorithm, so every engine
 * instance computes a shape the same way (bit-identical results across
 * processes). CUJEV_GEMM_TUNE=1 instead times the heuristic's candidates once
 * on the caller's buffers and stream (the output is simply rewritten) and
 * keeps the fastest; timing noise can then pick different algorithms in
 * different processes. */
static int tuning_enabled(void) {
    static int cached = -1;
    if (cached < 0) {
        const char *e = getenv("CUJEV_GEMM_TUNE");
        cached = e && *e == '1';
    }
    return cached;
}

static bool make_descs(int N, int M, int K, int f32out, GemmPlan &p) {
    const hipDataType out_t = f32out ? HIP_R_32F : HIP_R_16BF;
    if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return false;
    const int32_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof ta);
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof tb);
    return hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, K, M, K) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, K, N, K) == HIPBLAS_STATUS_SUCCESS &&
           hipblasLtMatrixLayoutCreate(&p.c, out_t, M, N, M) == HIPBLAS_STATUS_SUCCESS;
}

/* The tuned solution for (N, M, K, out): the entry for N itself, else the
 * one tuned for the nearest larger N, else the nearest smaller; used only if
 * hipBLASLt confirms it supports this exact problem. */
static bool table_algo(cujev_gemm *g, int N, int M, int K, int f32out, GemmPlan &p) {
    auto t = g->table.find(std::make_tuple(M, K, f32out));
    if (t == g->table.end() || t->second.empty())
        return false;
    auto it = t->second.lower_bound(N);
    if (it == t->second.end())
        --it;
    std::vector<int> idx{it->second};
    std::vector<hipblasLtMatmulHeuristicResult_t> res;
    if (hipblaslt_ext::getAlgosFromIndex(g->handle, idx, res) != HIPBLAS_STATUS_SUCCESS ||
        res.empty())
        return false;
    const float alpha = 1.f, beta = 0.f;
    size_t ws = 0;
    if (hipblaslt_ext::matmulIsAlgoSupported(g->handle, p.desc, &alpha, p.a, p.b, &beta, p.c, p.c,
                                             res[0].algo, ws) != HIPBLAS_STATUS_SUCCESS ||
        ws > g->ws_bytes)
        return false;
    p.algo = res[0].algo;
    p.ws = ws;
    return true;
}

/* Two timing events; false (and none left behind) when either cannot be made. */
static bool make_events(hipEvent_t &e0, hipEvent_t &e1) {
    e0 = e1 = nullptr;
    if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess)
        return true;
    if (e0)
        (void)hipEventDestroy(e0);
    e0 = e1 = nullptr;
    return false;
}

/* Records e1 on the stream, waits for it, and returns the milliseconds since
 * e0; negative when any of those steps fails. */
static float elapsed_ms(hipEvent_t e0, hipEvent_t e1, hipStream_t stream) {
    float ms = 0.f;
    if (hipEventRecord(e1, stream) != hipSuccess || hipEventSynchronize(e1) != hipSuccess ||
        hipEventElapsedTime(&ms, e0, e1) != hipSuccess)
        return -1.f;
    return ms;
}

static bool make_plan(cujev_gemm *g, int N, int M, int K, int f32out, GemmPlan &p, const void *X,
                      const void *W, void *Y, hipStream_t stream) {
    if (!make_descs(N, M, K, f32out, p))
        return false;
    const bool tuned = table_algo(g, N, M, K, f32out, p);
    if (getenv("CUJEV_GEMM_DEBUG"))
        fprintf(stderr, "[cujev] gemm plan N=%d M=%d K=%d f32out=%d: %s\n", N, M, K, f32out,
                tuned ? "tuned table" : "heuristic");
    if (tuned)
        return true;
    hipblasLtMatmulPreference_t pref;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS)
        return false;
    uint64_t ws = g->ws_bytes;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                          sizeof ws);
    constexpr int MAXC = 16;
    hipblasLtMatmulHeuristicResult_t res[MAXC];
    int count = 0;
    hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(
        g->handle, p.desc, p.a, p.b, p.c, p.c, pref, tuning_enabled() ? MAXC : 1, res, &count);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || count < 1)
        return false;
    int best = 0;
    hipEvent_t e0, e1;
    if (count > 1 && make_events(e0, e1)) {
        const float alpha = 1.f, beta = 0.f;
        float best_ms = 1e30f;
        for (int i = 0; i < count; i++) {
            if (res[i].state != HIPBLAS_STATUS_SUCCESS || res[i].workspaceSize > g->ws_bytes)
                continue;
            bool ok = true;
            for (int r = 0; r < 4 && ok; r++) {
                if (r == 1)
                    ok = hipEventRecord(e0, stream) == hipSuccess;
                ok = ok && hipblasLtMatmul(g->handle, p.desc, &alpha, W, p.a, X, p.b, &beta, Y,
                                           p.c, Y, p.c, &res[i].algo, g->workspace,
                                           res[i].workspaceSize, stream) == HIPBLAS_STATUS_SUCCESS;
            }
            const float ms = ok ? elapsed_ms(e0, e1, stream) : -1.f;
            if (ms >= 0.f && ms < best_ms) {
                best_ms = ms;
                best = i;
            }
        }
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
    }
    p.algo = res[best].algo;
    p.ws = res[best].workspaceSize;
    return true;
}

extern "C" hipError_t k_gemm(cujev_gemm *g, const bf16_t *X, const bf16_t *W, void *Y, int f32out,
                             int N, int M, int K, hipStream_t stream) {
    if (N <= 0)
        return hipSuccess;
    GemmPlan *plan;
    {
        std::lock_guard<std::mutex> lk(g->mu);
        auto key = std::make_tuple(N, M, K, f32out);
        auto it = g->plans.find(key);
        if (it == g->plans.end()) {
            GemmPlan p;
            if (!make_plan(g, N, M, K, f32out, p, X, W, Y, stream)) {
                destroy_plan(p);
                return hipErrorNotSupported;
            }
            it = g->plans.emplace(key, p).first;
        }
        plan = &it->second;
    }
    const float alpha = 1.f, beta = 0.f;
    hipblasStatus_t st = hipblasLtMatmul(g->handle, plan->desc, &alpha, W, plan->a, X, plan->b,
                                         &beta, Y, plan->c, Y, plan->c, &plan->algo, g->workspace,
                                         plan->ws, stream);
    return st == HIPBLAS_STATUS_SUCCESS ? hipSuccess : hipErrorLaunchFailure;
}

/* ---- tuned-algorithm table ------------------------------------------------
 * Text file: a header line "# hipblaslt <version>" and lines
 * "N M K f32out index" (index = hipBLASLt solution index, valid only for the
 * library version in the header). Returns the entries loaded, -1 when the
 * file cannot be read, -2 when it was made with another hipBLASLt version. */
extern "C" int cujev_gemm_load_table(cujev_gemm *g, const char *path) {
    FILE *f = path ? fopen(path, "r") : nullptr;
    if (!f)
        return -1;
    int ver = 0, file_ver = -1, n = 0;
    hipblasLtGetVersion(g->handle, &ver);
    char line[256];
    std::lock_guard<std::mutex> lk(g->mu);
    while (fgets(line, sizeof line, f)) {
        int N, M, K, o, idx;
        if (sscanf(line, "# hipblaslt %d", &file_ver) == 1)
            continue;
        if (line[0] == '#' || sscanf(line, "%d %d %d %d %d", &N, &M, &K, &o, &idx) != 5)
            continue;
        if (file_ver != ver) {
            fclose(f);
            g->table.clear();
            return -2;
        }
        g->table[std::make_tuple(M, K, o)][N] = idx;
        n++;
    }
    fclose(f);
    for (auto &kv : g->plans) /* plans made before the table are rebuilt */
        destroy_plan(kv.second);
    g->plans.clear();
    return n;
}

extern "C" int cujev_gemm_version(cujev_gemm *g) {
    int v = 0;
    hipblasLtGetVersion(g->handle, &v);
    return v;
}

/* Times every hipBLASLt solution that supports the problem (2 warm-up + 5
 * timed launches each, on the caller's buffers and stream; Y is rewritten)
 * and records the fastest in the table for this exact N. */
extern "C" int cujev_gemm_tune(cujev_gemm *g, const bf16_t *X, const bf16_t *W, void *Y, int f32out,
                               int N, int M, int K, hipStream_t stream, int *best_index,
                               float *best_us, float *heuristic_us) {
    std::lock_guard<std::mutex> lk(g->mu);
    std::vector<hipblasLtMatmulHeuristicResult_t> &all = g->all_algos[f32out];
    if (all.empty() &&
        hipblaslt_ext::getAllAlgos(g->handle, hipblaslt_ext::GemmType::HIPBLASLT_GEMM,
                                   HIPBLAS_OP_T, HIPBLAS_OP_N, HIP_R_16BF, HIP_R_16BF,
                                   f32out ? HIP_R_32F : HIP_R_16BF, f32out ? HIP_R_32F : HIP_R_16BF,
                                   HIPBLAS_COMPUTE_32F, all) != HIPBLAS_STATUS_SUCCESS)
        return -1;
    GemmPlan p;
    if (!make_descs(N, M, K, f32out, p)) {
        destroy_plan(p);
        return -1;
    }
    hipEvent_t e0, e1;
    if (!make_events(e0, e1)) {
        destroy_plan(p);
        return -1;
    }
    const float alpha = 1.f, beta = 0.f;
    auto time_algo = [&](hipblasLtMatmulAlgo_t &algo, size_t ws) -> float {
        for (int r = 0; r < 7; r++) {
            if (r == 2 && hipEventRecord(e0, stream) != hipSuccess)
                return -1.f;
            if (hipblasLtMatmul(g->handle, p.desc, &alpha, W, p.a, X, p.b, &beta, Y, p.c, Y, p.c,
                                &algo, g->workspace, ws, stream) != HIPBLAS_STATUS_SUCCESS)
                return -1.f;
        }
        const float ms = elapsed_ms(e0, e1, stream);
        return ms < 0.f ? -1.f : ms * 1e3f / 5.f;
    };
    /* the heuristic's own first choice, for reference */
    float heur = -1.f;
    hipblasLtMatmulPreference_t pref;
    if (hipblasLtMatmulPreferenceCreate(&pref) == HIPBLAS_STATUS_SUCCESS) {
        uint64_t wsb = g->ws_bytes;
        hipblasLtMatmulHeuristicResult_t top;
        int cnt = 0;
        if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES,
                                                  &wsb, sizeof wsb) == HIPBLAS_STATUS_SUCCESS &&
            hipblasLtMatmulAlgoGetHeuristic(g->handle, p.desc, p.a, p.b, p.c, p.c, pref, 1, &top,
                                            &cnt) == HIPBLAS_STATUS_SUCCESS && cnt > 0)
            heur = time_algo(top.algo, top.workspaceSize);
        hipblasLtMatmulPreferenceDestroy(pref);
    }
    float best = 1e30f;
    int best_i = -1;
    for (size_t i = 0; i < all.size(); i++) {
        size_t ws = 0;
        if (hipblaslt_ext::matmulIsAlgoSupported(g->handle, p.desc, &alpha, p.a, p.b, &beta, p.c,
                                                 p.c, all[i].algo, ws) !=
                HIPBLAS_STATUS_SUCCESS ||
            ws > g->ws_bytes)
            continue;
        const float t = time_algo(all[i].algo, ws);
        if (t > 0.f && t < best) {
            best = t;
            best_i = (int)i;
        }
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    destroy_plan(p);
    if (best_i < 0)
        return -1;
    *best_index = hipblaslt_ext::getIndexFromAlgo(all[best_i].algo);
    *best_us = best;
    *heuristic_us = heur;
    g->table[std::make_tuple(M, K, f32out)][N] = *best_index;
    auto pk = g->plans.find(std::make_tuple(N, M, K, f32out));
    if (pk != g->plans.end()) {
        destroy_plan(pk->second);
        g->plans.erase(pk);
    }
    return 0;
}
