// gemm.cpp -- row-major (batched) GEMM for the Linear / matmul ops, on hipBLASLt.
//
// The Linear layers of the GPT step are plain dense contractions, so they go
// to the vendor library rather than a hand-written kernel.  hipBLASLt picks
// gfx950 MFMA kernels; with fp32 operands it runs the fp32 matrix path
// (v_mfma_f32_*_f32), never a reduced-precision one.
//
// Row-major C[M,N] = alpha * op(A)[M,K] op(B)[K,N] + beta * C (+ bias[N] per
// row) is issued as the column-major product C^T = op(B)^T op(A)^T: a
// row-major matrix with leading dimension ld is the column-major transpose
// with the same ld, so no data moves.  Plans (descriptors, layouts and the
// heuristic's algorithm) are cached per problem; one hipBLASLt handle per
// device is created on first use and kept for the life of the process.
#include <hip/hip_runtime.h>
#include <hipblaslt/hipblaslt.h>

#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "kernels.h"

#include <string>

namespace inf {

namespace {

struct Key {
    int ta, tb, dt, bias, dev;
    int64_t M, N, K, lda, ldb, ldc, sa, sb, sc, batch;
    size_t ws;
    bool operator==(const Key& o) const { return std::memcmp(this, &o, sizeof(Key)) == 0; }
};

struct KeyHash {
    size_t operator()(const Key& k) const {
        const unsigned char* p = reinterpret_cast<const unsigned char*>(&k);
        size_t h = 1469598103934665603ull;
        for (size_t i = 0; i < sizeof(Key); ++i) h = (h ^ p[i]) * 1099511628211ull;
        return h;
    }
};

constexpr int kMaxAlgos = 16;

struct Plan {
    hipblasLtMatmulDesc_t desc = nullptr;
    hipblasLtMatrixLayout_t la = nullptr, lb = nullptr, lc = nullptr;
    hipblasLtMatmulAlgo_t algo[kMaxAlgos]{};
    int n_algo = 0;
    int cur = 0;  // the candidate in use: the first one that launched
    uint32_t reported = 0;  // candidates whose skip has been reported (bit i: candidate i)
};

std::mutex g_mu;
std::vector<hipblasLtHandle_t>* g_handles = new std::vector<hipblasLtHandle_t>();
std::unordered_map<Key, Plan, KeyHash>* g_plans = new std::unordered_map<Key, Plan, KeyHash>();

hipblasLtHandle_t handle_for(int dev) {
    if ((int)g_handles->size() <= dev) g_handles->resize((size_t)dev + 1, nullptr);
    hipblasLtHandle_t& h = (*g_handles)[(size_t)dev];
    if (!h && hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) h = nullptr;
    return h;
}

bool set_layout(hipblasLtMatrixLayout_t* l, hipDataType t, uint64_t rows, uint64_t cols, int64_t ld, int64_t batch,
                int64_t stride) {
    if (hipblasLtMatrixLayoutCreate(l, t, rows, cols, ld) != HIPBLAS_STATUS_SUCCESS) return false;
    if (batch > 1) {
        const int32_t bc = (int32_t)batch;
        if (hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_BATCH_COUNT, &bc, sizeof(bc)) !=
            HIPBLAS_STATUS_SUCCESS)
            return false;
        if (hipblasLtMatrixLayoutSetAttribute(*l, HIPBLASLT_MATRIX_LAYOUT_STRIDED_BATCH_OFFSET, &stride,
                                              sizeof(stride)) != HIPBLAS_STATUS_SUCCESS)
            return false;
    }
    return true;
}

void destroy(Plan& p) {
    if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
    if (p.lb) hipblasLtMatrixLayoutDestroy(p.lb);
    if (p.lc) hipblasLtMatrixLayoutDestroy(p.lc);
    if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
    p = Plan{};
}

// Column-major view of the row-major problem: m' = N, n' = M, k' = K,
// A' = B (op' = T iff tb), B' = A (op' = T iff ta), D' = C^T.
int make_plan(hipblasLtHandle_t h, const Key& k, Plan& p) {
    const hipDataType t = k.dt ? HIP_R_16BF : HIP_R_32F;
    if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return 1;
    const int32_t opa = k.tb ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    const int32_t opb = k.ta ? HIPBLAS_OP_T : HIPBLAS_OP_N;
    if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opa, sizeof(opa)) ||
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opb, sizeof(opb)))
        return 1;
    if (k.bias) {
        const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
        const int32_t bt = t;
        if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) ||
            hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bt, sizeof(bt)))
            return 1;
    }
    // stored shapes (rows x cols, column-major) of A' = B and B' = A
    const uint64_t ar = k.tb ? (uint64_t)k.K : (uint64_t)k.N, ac = k.tb ? (uint64_t)k.N : (uint64_t)k.K;
    const uint64_t br = k.ta ? (uint64_t)k.M : (uint64_t)k.K, bc = k.ta ? (uint64_t)k.K : (uint64_t)k.M;
    if (!set_layout(&p.la, t, ar, ac, k.ldb, k.batch, k.sb) || !set_layout(&p.lb, t, br, bc, k.lda, k.batch, k.sa) ||
        !set_layout(&p.lc, t, (uint64_t)k.N, (uint64_t)k.M, k.ldc, k.batch, k.sc))
        return 1;
    hipblasLtMatmulPreference_t pref = nullptr;
    if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return 1;
    const uint64_t wsmax = k.ws;
    hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &wsmax, sizeof(wsmax));
    hipblasLtMatmulHeuristicResult_t res[kMaxAlgos];
    int n = 0;
    const hipblasStatus_t st =
        hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.la, p.lb, p.lc, p.lc, pref, kMaxAlgos, res, &n);
    hipblasLtMatmulPreferenceDestroy(pref);
    if (st != HIPBLAS_STATUS_SUCCESS || n < 1) return 2;
    for (int i = 0; i < n && i < kMaxAlgos; ++i)
        if (res[i].state == HIPBLAS_STATUS_SUCCESS) p.algo[p.n_algo++] = res[i].algo;
    return p.n_algo ? 0 : 2;
}

}  // namespace

int launch_gemm(const GemmArgs& g, hipStream_t s) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        set_error_detail("inf_gemm: hipGetDevice failed");
        return 1;
    }
    // An error left pending by an earlier HIP call on this thread fails the
    // call with that error named (nothing is launched): hipBLASLt would
    // otherwise report it as its own failure, or the caller would never see it.
    const hipError_t pending = hipGetLastError();
    if (pending != hipSuccess) {
        set_error_detail(std::string("inf_gemm: HIP error pending from an earlier call: ") + hipGetErrorName(pending) +
                         " (" + hipGetErrorString(pending) + "); nothing launched");
        return 1;
    }
    Key k;
    std::memset(&k, 0, sizeof(k));  // padding bytes take part in hashing / comparison
    k.ta = g.ta;
    k.tb = g.tb;
    k.dt = g.bf16;
    k.bias = g.bias != nullptr;
    k.dev = dev;
    k.M = g.M;
    k.N = g.N;
    k.K = g.K;
    k.lda = g.lda;
    k.ldb = g.ldb;
    k.ldc = g.ldc;
    k.sa = g.batch > 1 ? g.sa : 0;
    k.sb = g.batch > 1 ? g.sb : 0;
    k.sc = g.batch > 1 ? g.sc : 0;
    k.batch = g.batch;
    k.ws = g.ws_bytes;
    std::lock_guard<std::mutex> lk(g_mu);
    char shape[192];
    std::snprintf(shape, sizeof(shape), "M=%lld N=%lld K=%lld ta=%d tb=%d lda=%lld ldb=%lld ldc=%lld batch=%lld bias=%d",
                  (long long)g.M, (long long)g.N, (long long)g.K, g.ta, g.tb, (long long)g.lda, (long long)g.ldb,
                  (long long)g.ldc, (long long)g.batch, g.bias != nullptr);
    hipblasLtHandle_t h = handle_for(dev);
    if (!h) {
        set_error_detail("inf_gemm: hipblasLtCreate failed");
        return 1;
    }
    auto it = g_plans->find(k);
    if (it == g_plans->end()) {
        Plan p;
        const int e = make_plan(h, k, p);
        if (e) {
            destroy(p);
            set_error_detail(std::string("inf_gemm: ") + (e == 2 ? "no hipBLASLt algorithm" : "descriptor setup failed") +
                             " for " + shape);
            return e == 2 ? 2 : 1;
        }
        it = g_plans->emplace(k, p).first;
    }
    Plan& p = it->second;
    if (g.bias) {
        const void* bp = g.bias;
        if (hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp))) {
            set_error_detail(std::string("inf_gemm: setting the bias pointer failed for ") + shape);
            return 1;
        }
    }
    const float alpha = g.alpha, beta = g.beta;
    // The heuristic's candidates in order, starting from the one in use: a
    // candidate the installed library cannot launch (some builds return
    // HIPBLAS_STATUS_INTERNAL_ERROR for a listed solution) is skipped for good,
    // and each skip is reported once, on stderr and in the call's detail string.
    hipblasStatus_t st = HIPBLAS_STATUS_NOT_SUPPORTED;
    std::string skipped;
    for (; p.cur < p.n_algo; ++p.cur) {
        st = hipblasLtMatmul(h, p.desc, &alpha, g.B, p.la, g.A, p.lb, &beta, g.C, p.lc, g.C, p.lc, &p.algo[p.cur],
                             g.ws, g.ws_bytes, s);
        if (st == HIPBLAS_STATUS_SUCCESS) break;
        const hipError_t le = hipGetLastError();  // the failed launch's own error, if it left one
        const uint32_t bit = 1u << p.cur;
        if (!(p.reported & bit)) {
            p.reported |= bit;
            char line[160];
            std::snprintf(line, sizeof(line), "candidate %d of %d skipped (hipblasLtMatmul status %d, HIP %s); ",
                          p.cur + 1, p.n_algo, (int)st, hipGetErrorName(le));
            skipped += line;
            std::fprintf(stderr, "inferno_hip: inf_gemm: %sfor %s\n", line, shape);
        }
    }
    if (st != HIPBLAS_STATUS_SUCCESS) {
        p.cur = 0;  // all failed: start over on the next call
        set_error_detail(std::string("inf_gemm: hipblasLtMatmul status ") + std::to_string((int)st) + " for " + shape +
                         " with every one of " + std::to_string(p.n_algo) + " heuristic candidates; " + skipped);
        return 1;
    }
    if (!skipped.empty()) set_error_detail("inf_gemm: " + skipped + "for " + shape);
    return 0;
}

}  // namespace inf
