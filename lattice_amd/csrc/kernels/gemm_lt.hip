// Plain projection GEMM through hipBLASLt for many tokens (M > 128), where the
// library's MFMA tiling is faster than the weight-stream kernel of gemm.hip
// (which stays in charge of every decode-sized, split or fused GEMM).
//
// Y[M][N] = X[M][K] W[N][K]^T in row-major terms is, column-major,
// Y^T[N][M] = op(W) X^T with W stored as a K x N column-major matrix
// (transposed by the op) and X as a K x M one: m = N, n = M, k = K.
// bf16 operands and result, fp32 compute.
//
// The first call of a shape times the library's top candidates (up to
// kLtCandidates, 2 + 5 runs each on the caller's stream, HIP events) and
// keeps the fastest for the process; that call synchronizes the stream.
// KCMM_GEMM_LT_TUNE=0 takes the heuristic's first choice instead.
#include <hipblaslt/hipblaslt.h>

#include <algorithm>
#include <cstdlib>
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "../device_api.hpp"
#include "common.hpp"

namespace kcmm {
namespace {

constexpr size_t kLtWorkspace = 32u << 20;   // bytes offered to the heuristic
constexpr int kLtCandidates = 8;

struct LtPlan {
    bool ok = false;
    bool tuned = false;
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t a = nullptr, b = nullptr, c = nullptr;
    hipblasLtMatmulAlgo_t algo{};
    size_t workspace = 0;
    std::vector<hipblasLtMatmulHeuristicResult_t> cands;
};

struct LtState {
    std::mutex mu;
    std::map<int, hipblasLtHandle_t> handles;                              // per device
    std::map<std::tuple<int, uint32_t, uint32_t, uint32_t>, LtPlan> plans;
};

int env_int_lt(const char* name, int dflt) {
    const char* e = std::getenv(name);
    return e ? std::atoi(e) : dflt;
}

LtState& state() {
    static LtState* s = new LtState();   // kept for the process lifetime
    return *s;
}

bool make_plan(hipblasLtHandle_t h, uint32_t m, uint32_t n, uint32_t k, LtPlan* p) {
    const hipblasOperation_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
    if (hipblasLtMatmulDescCreate(&p->desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
        return false;
    if (hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(p->desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)) !=
            HIPBLAS_STATUS_SUCCESS)
        return false;
    if (hipblasLtMatrixLayoutCreate(&p->a, HIP_R_16BF, k, n, k) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p->b, HIP_R_16BF, k, m, k) != HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatrixLayoutCreate(&p->c, HIP_R_16BF, n, m, n) != HIPBLAS_STATUS_SUCCESS)
        return false;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
    const uint64_t ws = kLtWorkspace;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws,
                                          sizeof(ws));
    hipblasLtMatmulHeuristicResult_t res[kLtCandidates] = {};
    int returned = 0;
    const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(h, p->desc, p->a, p->b, p->c, p->c,
                                                               pref, kLtCandidates, res, &returned);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || returned < 1) return false;
    p->algo = res[0].algo;
    p->workspace = res[0].workspaceSize;
    for (int i = 0; i < returned; ++i)
        if (res[i].state == HIPBLAS_STATUS_SUCCESS) p->cands.push_back(res[i]);
    return true;
}

}  // namespace

namespace dev {

bool lt_gemm_bf16(uint64_t x, uint64_t w, uint64_t y, uint32_t m, uint32_t n, uint32_t k,
                  uint64_t stream, bool* used, std::string* err) {
    *used = false;
    int device = 0;
    KCMM_HIP_CHECK(hipGetDevice(&device), err);
    LtState& s = state();
    hipblasLtHandle_t h = nullptr;
    LtPlan plan;
    {
        std::lock_guard<std::mutex> lk(s.mu);
        auto hit = s.handles.find(device);
        if (hit == s.handles.end()) {
            if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) h = nullptr;
            s.handles[device] = h;
        } else {
            h = hit->second;
        }
        if (h == nullptr) return true;   // no library on this device: the caller's kernel runs
        const auto key = std::make_tuple(device, m, n, k);
        auto it = s.plans.find(key);
        if (it == s.plans.end()) {
            LtPlan p;
            p.ok = make_plan(h, m, n, k, &p);
            it = s.plans.emplace(key, p).first;
        }
        plan = it->second;
    }
    if (!plan.ok) return true;
    const float alpha = 1.0f, beta = 0.0f;
    hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
    auto run = [&](const hipblasLtMatmulAlgo_t& algo, void* ws, size_t wsz) {
        return hipblasLtMatmul(h, plan.desc, &alpha, reinterpret_cast<const void*>(w), plan.a,
                               reinterpret_cast<const void*>(x), plan.b, &beta,
                               reinterpret_cast<const void*>(y), plan.c, reinterpret_cast<void*>(y),
                               plan.c, &algo, ws, wsz, hs);
    };
    if (!plan.tuned && plan.cands.size() > 1 && env_int_lt("KCMM_GEMM_LT_TUNE", 1) != 0) {
        // time the candidates once for this shape and keep the fastest
        size_t wmax = 0;
        for (const auto& c : plan.cands) wmax = std::max(wmax, c.workspaceSize);
        void* tws = nullptr;
        if (wmax > 0 && !stream_workspace(stream, 5, wmax, &tws, false, err)) return false;
        hipEvent_t e0, e1;
        KCMM_HIP_CHECK(hipEventCreate(&e0), err);
        KCMM_HIP_CHECK(hipEventCreate(&e1), err);
        float best = 0.0f;
        size_t pick = 0;
        for (size_t i = 0; i < plan.cands.size(); ++i) {
            const auto& c = plan.cands[i];
            bool ok = run(c.algo, tws, c.workspaceSize) == HIPBLAS_STATUS_SUCCESS &&
                      run(c.algo, tws, c.workspaceSize) == HIPBLAS_STATUS_SUCCESS;
            if (!ok) continue;
            (void)hipEventRecord(e0, hs);
            for (int r = 0; r < 5 && ok; ++r)
                ok = run(c.algo, tws, c.workspaceSize) == HIPBLAS_STATUS_SUCCESS;
            (void)hipEventRecord(e1, hs);
            if (!ok || hipEventSynchronize(e1) != hipSuccess) continue;
            float ms = 0.0f;
            if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) continue;
            if (best == 0.0f || ms < best) {
                best = ms;
                pick = i;
            }
        }
        (void)hipEventDestroy(e0);
        (void)hipEventDestroy(e1);
        (void)hipGetLastError();
        plan.algo = plan.cands[pick].algo;
        plan.workspace = plan.cands[pick].workspaceSize;
        plan.tuned = true;
        std::lock_guard<std::mutex> lk(s.mu);
        LtPlan& stored = s.plans[std::make_tuple(device, m, n, k)];
        stored.algo = plan.algo;
        stored.workspace = plan.workspace;
        stored.tuned = true;
    }
    void* ws = nullptr;
    if (plan.workspace > 0 && !stream_workspace(stream, 5, plan.workspace, &ws, false, err))
        return false;
    const hipblasStatus_t st = run(plan.algo, ws, plan.workspace);
    if (st != HIPBLAS_STATUS_SUCCESS) {
        *err = "hipblasLtMatmul failed (status " + std::to_string(static_cast<int>(st)) + ")";
        return false;
    }
    *used = true;
    return true;
}

}  // namespace dev
}  // namespace kcmm
