// rocsparse_baseline.cpp -- the vendor comparison: hipSPARSE SpMM on the same CSR, B and C.
//
// Same library calls and precision pairing as the reference's baseline (src/kernels.cu:60-206:
// CSR int32, row-major dense B and C, FP32 compute; the FP16 variant has binary16 A values and
// B with FP32 C and alpha = the range scale).  Descriptor creation, buffer sizing and
// hipsparseSpMM_preprocess run once per distinct argument set and are reported as setup;
// only hipsparseSpMM sits between the timing events.
#include <hip/hip_runtime.h>
#include <hipsparse/hipsparse.h>

#include <chrono>
#include <cstdio>

#include "vcsrmc_bench.h"

namespace {

struct Ctx {
    hipsparseHandle_t handle = nullptr;
    hipsparseSpMatDescr_t A = nullptr;
    hipsparseDnMatDescr_t B = nullptr, C = nullptr;
    void* buffer = nullptr;
    size_t buffer_bytes = 0;
    const void *k_rp = nullptr, *k_col = nullptr, *k_val = nullptr, *k_B = nullptr, *k_C = nullptr;
    int k_M = -1, k_N = -1, k_nnz = -1, k_O = -1, k_vf16 = -1, k_bf16 = -1, k_alg = -1;
    float setup_ms = 0.f;
    void drop_descr() {
        if (A) hipsparseDestroySpMat(A);
        if (B) hipsparseDestroyDnMat(B);
        if (C) hipsparseDestroyDnMat(C);
        A = nullptr; B = nullptr; C = nullptr;
    }
};

Ctx g_ctx;

hipsparseSpMMAlg_t alg_of(int alg) {
    switch (alg) {
        case 1: return HIPSPARSE_SPMM_CSR_ALG1;
        case 2: return HIPSPARSE_SPMM_CSR_ALG2;
        case 3: return HIPSPARSE_SPMM_CSR_ALG3;
        default: return HIPSPARSE_SPMM_ALG_DEFAULT;
    }
}

}  // namespace

#define SP(call)                                                                              \
    do {                                                                                      \
        const hipsparseStatus_t s_ = (call);                                                  \
        if (s_ != HIPSPARSE_STATUS_SUCCESS) {                                                 \
            std::fprintf(stderr, "hipSPARSE %s failed: status %d\n", #call, (int)s_);         \
            return 10 + (int)s_;                                                              \
        }                                                                                     \
    } while (0)
#define HP(call)                                                                              \
    do {                                                                                      \
        const hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) {                                                               \
            std::fprintf(stderr, "HIP %s failed: %s\n", #call, hipGetErrorString(e_));        \
            return 2;                                                                         \
        }                                                                                     \
    } while (0)

extern "C" {

int vcsrmc_rocsparse_spmm(int M, int N, int nnz, const int* d_row_ptr, const int* d_col,
                          const void* d_val, int val_f16, const void* d_B, int b_f16, int O,
                          float* d_C, float alpha, int alg, void* stream, float* ms,
                          float* setup_ms) {
    Ctx& c = g_ctx;
    hipStream_t st = (hipStream_t)stream;
    if (!c.handle) SP(hipsparseCreate(&c.handle));
    SP(hipsparseSetStream(c.handle, st));
    const hipsparseSpMMAlg_t a = alg_of(alg);
    const float beta = 0.f;
    const bool same = c.A && c.k_rp == d_row_ptr && c.k_col == d_col && c.k_val == d_val &&
                      c.k_B == d_B && c.k_C == d_C && c.k_M == M && c.k_N == N &&
                      c.k_nnz == nnz && c.k_O == O && c.k_vf16 == val_f16 && c.k_bf16 == b_f16 &&
                      c.k_alg == alg;
    if (!same) {
        c.drop_descr();
        const auto t0 = std::chrono::steady_clock::now();
        SP(hipsparseCreateCsr(&c.A, M, N, nnz, (void*)d_row_ptr, (void*)d_col, (void*)d_val,
                              HIPSPARSE_INDEX_32I, HIPSPARSE_INDEX_32I, HIPSPARSE_INDEX_BASE_ZERO,
                              val_f16 ? HIP_R_16F : HIP_R_32F));
        SP(hipsparseCreateDnMat(&c.B, N, O, O, (void*)d_B, b_f16 ? HIP_R_16F : HIP_R_32F,
                                HIPSPARSE_ORDER_ROW));
        SP(hipsparseCreateDnMat(&c.C, M, O, O, (void*)d_C, HIP_R_32F, HIPSPARSE_ORDER_ROW));
        size_t bytes = 0;
        SP(hipsparseSpMM_bufferSize(c.handle, HIPSPARSE_OPERATION_NON_TRANSPOSE,
                                    HIPSPARSE_OPERATION_NON_TRANSPOSE, &alpha, c.A, c.B, &beta, c.C,
                                    HIP_R_32F, a, &bytes));
        if (bytes > c.buffer_bytes) {
            if (c.buffer) HP(hipFree(c.buffer));
            c.buffer = nullptr;
            HP(hipMalloc(&c.buffer, bytes));
            c.buffer_bytes = bytes;
        }
        SP(hipsparseSpMM_preprocess(c.handle, HIPSPARSE_OPERATION_NON_TRANSPOSE,
                                    HIPSPARSE_OPERATION_NON_TRANSPOSE, &alpha, c.A, c.B, &beta,
                                    c.C, HIP_R_32F, a, c.buffer));
        HP(hipStreamSynchronize(st));
        c.setup_ms = std::chrono::duration<float, std::milli>(std::chrono::steady_clock::now() - t0)
                         .count();
        c.k_rp = d_row_ptr; c.k_col = d_col; c.k_val = d_val; c.k_B = d_B; c.k_C = d_C;
        c.k_M = M; c.k_N = N; c.k_nnz = nnz; c.k_O = O; c.k_vf16 = val_f16; c.k_bf16 = b_f16;
        c.k_alg = alg;
    }
    if (setup_ms) *setup_ms = c.setup_ms;
    hipEvent_t e0, e1;
    HP(hipEventCreate(&e0));
    HP(hipEventCreate(&e1));
    HP(hipEventRecord(e0, st));
    SP(hipsparseSpMM(c.handle, HIPSPARSE_OPERATION_NON_TRANSPOSE, HIPSPARSE_OPERATION_NON_TRANSPOSE,
                     &alpha, c.A, c.B, &beta, c.C, HIP_R_32F, a, c.buffer));
    HP(hipEventRecord(e1, st));
    HP(hipEventSynchronize(e1));
    float t = 0.f;
    HP(hipEventElapsedTime(&t, e0, e1));
    HP(hipEventDestroy(e0));
    HP(hipEventDestroy(e1));
    if (ms) *ms = t;
    return 0;
}

int vcsrmc_rocsparse_release(void) {
    Ctx& c = g_ctx;
    c.drop_descr();
    if (c.buffer) (void)hipFree(c.buffer);
    if (c.handle) hipsparseDestroy(c.handle);
    c = Ctx();
    return 0;
}

}  // extern "C"
