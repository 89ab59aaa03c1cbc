// rocsparse_baseline.cpp -- the vendor comparison: hipSPARSE SpMM on the same CSR, B and C.
//
// The library calls and precision pairing are those of the reference's baseline
// (src/kernels.cu:60-206): CSR with int32 indices, row-major dense B and C, FP32 compute, beta 0;
// its FP16 variant has binary16 A values and B with FP32 C and alpha = the range scale.
//
// Organisation: a Plan is everything hipSPARSE needs for one argument set (descriptors, a
// workspace analysed by hipsparseSpMM_preprocess, a pair of timing events), built once and
// reported as setup time; a Session keeps the handle and the few most recent plans, so that
// alternating FP32 and FP16 comparisons on one matrix reuse both analyses.  Only hipsparseSpMM
// sits between a plan's timing events.
#include <hip/hip_runtime.h>
#include <hipsparse/hipsparse.h>

#include <chrono>
#include <cstdio>
#include <memory>
#include <vector>

#include "vcsrmc_bench.h"

namespace {

// A failed library call, carrying the status the C ABI returns (2: HIP, 10 + s: hipSPARSE s).
struct Failure {
    int code;
};

void hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    std::fprintf(stderr, "HIP %s failed: %s\n", what, hipGetErrorString(e));
    throw Failure{2};
}

void sparse_ok(hipsparseStatus_t s, const char* what) {
    if (s == HIPSPARSE_STATUS_SUCCESS) return;
    std::fprintf(stderr, "hipSPARSE %s failed: status %d\n", what, (int)s);
    throw Failure{10 + (int)s};
}

// Everything that fixes the descriptors and the analysis.
struct PlanKey {
    int M, N, nnz, O;
    const void *row_ptr, *col, *val, *B;
    float* C;
    bool val_f16, b_f16;
    int alg;
    bool operator==(const PlanKey& o) const {
        return M == o.M && N == o.N && nnz == o.nnz && O == o.O && row_ptr == o.row_ptr &&
               col == o.col && val == o.val && B == o.B && C == o.C && val_f16 == o.val_f16 &&
               b_f16 == o.b_f16 && alg == o.alg;
    }
};

hipsparseSpMMAlg_t algorithm(int alg) {
    if (alg == 1) return HIPSPARSE_SPMM_CSR_ALG1;
    if (alg == 2) return HIPSPARSE_SPMM_CSR_ALG2;
    if (alg == 3) return HIPSPARSE_SPMM_CSR_ALG3;
    return HIPSPARSE_SPMM_ALG_DEFAULT;
}

class Plan {
public:
    explicit Plan(const PlanKey& k) : key(k) {}

    // Builds the descriptors and analyses the product on `st` (each run passes its own alpha).
    // On failure the destructor releases whatever was created.
    void build(hipsparseHandle_t h, float alpha, hipStream_t st) {
        const PlanKey& k = key;
        const auto start = std::chrono::steady_clock::now();
        sparse_ok(hipsparseCreateCsr(&A_, k.M, k.N, k.nnz, const_cast<void*>(k.row_ptr),
                                     const_cast<void*>(k.col), const_cast<void*>(k.val),
                                     HIPSPARSE_INDEX_32I, HIPSPARSE_INDEX_32I,
                                     HIPSPARSE_INDEX_BASE_ZERO, k.val_f16 ? HIP_R_16F : HIP_R_32F),
                  "CreateCsr");
        sparse_ok(hipsparseCreateDnMat(&B_, k.N, k.O, k.O, const_cast<void*>(k.B),
                                       k.b_f16 ? HIP_R_16F : HIP_R_32F, HIPSPARSE_ORDER_ROW),
                  "CreateDnMat(B)");
        sparse_ok(hipsparseCreateDnMat(&C_, k.M, k.O, k.O, k.C, HIP_R_32F, HIPSPARSE_ORDER_ROW),
                  "CreateDnMat(C)");
        const float beta = 0.f;
        size_t bytes = 0;
        sparse_ok(hipsparseSpMM_bufferSize(h, HIPSPARSE_OPERATION_NON_TRANSPOSE,
                                           HIPSPARSE_OPERATION_NON_TRANSPOSE, &alpha, A_, B_,
                                           &beta, C_, HIP_R_32F, algorithm(k.alg), &bytes),
                  "SpMM_bufferSize");
        if (bytes) hip_ok(hipMalloc(&work_, bytes), "hipMalloc(workspace)");
        sparse_ok(hipsparseSpMM_preprocess(h, HIPSPARSE_OPERATION_NON_TRANSPOSE,
                                           HIPSPARSE_OPERATION_NON_TRANSPOSE, &alpha, A_, B_,
                                           &beta, C_, HIP_R_32F, algorithm(k.alg), work_),
                  "SpMM_preprocess");
        hip_ok(hipStreamSynchronize(st), "hipStreamSynchronize");
        hip_ok(hipEventCreate(&t0_), "hipEventCreate");
        hip_ok(hipEventCreate(&t1_), "hipEventCreate");
        setup_ms = std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() -
                                                            start).count();
    }
    ~Plan() {
        if (t1_) (void)hipEventDestroy(t1_);
        if (t0_) (void)hipEventDestroy(t0_);
        if (work_) (void)hipFree(work_);
        if (C_) (void)hipsparseDestroyDnMat(C_);
        if (B_) (void)hipsparseDestroyDnMat(B_);
        if (A_) (void)hipsparseDestroySpMat(A_);
    }
    Plan(const Plan&) = delete;
    Plan& operator=(const Plan&) = delete;

    // One product between this plan's events; returns its time in milliseconds.
    float run_timed(hipsparseHandle_t h, float alpha, hipStream_t st) {
        const float beta = 0.f;
        hip_ok(hipEventRecord(t0_, st), "hipEventRecord");
        sparse_ok(hipsparseSpMM(h, HIPSPARSE_OPERATION_NON_TRANSPOSE,
                                HIPSPARSE_OPERATION_NON_TRANSPOSE, &alpha, A_, B_, &beta, C_,
                                HIP_R_32F, algorithm(key.alg), work_),
                  "SpMM");
        hip_ok(hipEventRecord(t1_, st), "hipEventRecord");
        hip_ok(hipEventSynchronize(t1_), "hipEventSynchronize");
        float ms = 0.f;
        hip_ok(hipEventElapsedTime(&ms, t0_, t1_), "hipEventElapsedTime");
        return ms;
    }

    const PlanKey key;
    float setup_ms = 0.f;

private:
    hipsparseSpMatDescr_t A_ = nullptr;
    hipsparseDnMatDescr_t B_ = nullptr, C_ = nullptr;
    void* work_ = nullptr;
    hipEvent_t t0_ = nullptr, t1_ = nullptr;
};

class Session {
public:
    static constexpr size_t kPlans = 4;

    // The plan for `k`, most recent first; a new plan evicts the least recently used one.
    Plan& plan(const PlanKey& k, float alpha, hipStream_t st) {
        if (!handle_) sparse_ok(hipsparseCreate(&handle_), "Create");
        for (size_t i = 0; i < plans_.size(); ++i)
            if (plans_[i]->key == k) {
                std::unique_ptr<Plan> p = std::move(plans_[i]);
                plans_.erase(plans_.begin() + (long)i);
                plans_.insert(plans_.begin(), std::move(p));
                return *plans_.front();
            }
        if (plans_.size() == kPlans) plans_.pop_back();
        sparse_ok(hipsparseSetStream(handle_, st), "SetStream");
        auto p = std::make_unique<Plan>(k);
        p->build(handle_, alpha, st);
        plans_.insert(plans_.begin(), std::move(p));
        return *plans_.front();
    }
    hipsparseHandle_t handle() const { return handle_; }
    void release() {
        plans_.clear();
        if (handle_) (void)hipsparseDestroy(handle_);
        handle_ = nullptr;
    }

private:
    hipsparseHandle_t handle_ = nullptr;
    std::vector<std::unique_ptr<Plan>> plans_;
};

// Plans are keyed by device addresses, as the reference's cache is: a caller that frees and
// reallocates operands of the same sizes calls vcsrmc_rocsparse_release first.  The session is
// never destroyed (releasing HIP objects during static destruction can outlive the runtime).
Session& session() {
    static Session* s = new Session;
    return *s;
}

}  // namespace

extern "C" {

int vcsrmc_rocsparse_spmm(int M, int N, int nnz, const int* d_row_ptr, const int* d_col,
                          const void* d_val, int val_f16, const void* d_B, int b_f16, int O,
                          float* d_C, float alpha, int alg, void* stream, float* ms,
                          float* setup_ms) {
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const PlanKey key{M, N, nnz, O, d_row_ptr, d_col, d_val, d_B, d_C, val_f16 != 0, b_f16 != 0,
                      alg};
    try {
        Session& s = session();
        Plan& p = s.plan(key, alpha, st);
        sparse_ok(hipsparseSetStream(s.handle(), st), "SetStream");
        const float t = p.run_timed(s.handle(), alpha, st);
        if (setup_ms) *setup_ms = p.setup_ms;
        if (ms) *ms = t;
        return 0;
    } catch (const Failure& f) {
        return f.code;
    } catch (...) {
        return 1;
    }
}

int vcsrmc_rocsparse_release(void) {
    session().release();
    return 0;
}

}  // extern "C"
