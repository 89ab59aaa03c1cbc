// vcsr_formats.hip -- the reference's C++ surface (include/vcsr_formats.hpp, include/reorder.hpp)
// over the C ABI.
#include <cstdio>
#include <cstdlib>
#include <stdexcept>
#include <string>

#include "../../include/reorder.hpp"
#include "../../include/vcsr_formats.hpp"
#include "../../include/vcsrmc.h"

namespace {

vcsrmc_t g_handle = nullptr;  // the one device-resident format (src/vcsr_mc.cu:126-131)
bool g_uploaded = false;

// Runtime failures end the process, as CUDA_CHECK does (include/cuda_check.hpp:7-14);
// argument and format errors become std::runtime_error.
void check(int status, const char* what) {
    if (status == VCSRMC_OK) return;
    if (status == VCSRMC_ERR_HIP) {
        std::fprintf(stderr, "HIP error in %s: %s\n", what, vcsrmc_last_error());
        std::exit(EXIT_FAILURE);
    }
    throw std::runtime_error(std::string(what) + ": " + vcsrmc_last_error());
}

void hip_check(hipError_t e, const char* what) {
    if (e == hipSuccess) return;
    std::fprintf(stderr, "HIP error in %s: %s\n", what, hipGetErrorString(e));
    std::exit(EXIT_FAILURE);
}

template <typename T>
struct Dev {
    T* p = nullptr;
    explicit Dev(const std::vector<T>& h) {
        hip_check(hipMalloc((void**)&p, sizeof(T) * (h.size() ? h.size() : 1)), "hipMalloc");
        if (!h.empty())
            hip_check(hipMemcpy(p, h.data(), sizeof(T) * h.size(), hipMemcpyHostToDevice),
                      "hipMemcpy");
    }
    explicit Dev(size_t n) {
        hip_check(hipMalloc((void**)&p, sizeof(T) * (n ? n : 1)), "hipMalloc");
    }
    ~Dev() { if (p) (void)hipFree(p); }
    void to_host(std::vector<T>& h) const {
        if (!h.empty())
            hip_check(hipMemcpy(h.data(), p, sizeof(T) * h.size(), hipMemcpyDeviceToHost),
                      "hipMemcpy");
    }
};

}  // namespace

float half_scale(const CSR& csr) {
    Dev<float> v(csr.val);
    float s = 1.0f;
    check(vcsrmc_half_scale(v.p, (long long)csr.val.size(), &s, nullptr), "half_scale");
    return s;
}

VCSRMC csr_to_vcsr_mc(const CSR& csr, bool fp32, int segw) {
    if (segw != 16 && segw != 32 && segw != 48 && segw != 64)
        throw std::runtime_error("vcsr_mc supports segw in {16, 32, 48, 64}");
    Dev<int> rp(csr.row_ptr), ci(csr.col);
    Dev<float> vv(csr.val);
    vcsrmc_t h = nullptr;
    check(vcsrmc_create(&h), "csr_to_vcsr_mc");
    VCSRMC V;
    try {
        check(vcsrmc_build_csr(h, rp.p, ci.p, vv.p, csr.M, csr.N, csr.nnz, fp32 ? 1 : 0, segw,
                               nullptr),
              "csr_to_vcsr_mc");
        vcsrmc_info info;
        check(vcsrmc_get_info(h, &info), "csr_to_vcsr_mc");
        V.M = info.M; V.N = info.N; V.segw = info.segw; V.bundle = info.bundle;
        V.num_segments = info.num_segments; V.scale = info.scale; V.fp32 = info.fp32 != 0;
        V.group_ptr.resize((size_t)info.num_groups + 1);
        V.group_depth.resize(info.num_groups);
        V.group_seg_base.resize(info.num_groups);
        V.group_rows.resize((size_t)16 * info.num_groups);
        V.lcol.resize(info.nval);
        V.val.resize(info.nval);
        V.item_gbeg.resize(info.num_items);
        V.item_gend.resize(info.num_items);
        check(vcsrmc_download(h, V.group_ptr.data(), V.group_depth.data(), V.group_seg_base.data(),
                              V.group_rows.data(), V.lcol.data(), V.val.data(), V.item_gbeg.data(),
                              V.item_gend.data()),
              "csr_to_vcsr_mc");
    } catch (...) {
        vcsrmc_destroy(h);
        throw;
    }
    check(vcsrmc_destroy(h), "csr_to_vcsr_mc");
    return V;
}

void upload_vcsr_mc_device(const VCSRMC& V) {
    if (g_uploaded) return;
    // The C ABI takes sizes and pointers; the vectors must hold what those sizes say.
    const size_t G = V.group_depth.size();
    if (V.group_ptr.size() != G + 1 || V.group_seg_base.size() != G ||
        V.group_rows.size() != 16 * G || V.lcol.size() != V.val.size() ||
        V.item_gend.size() != V.item_gbeg.size())
        throw std::runtime_error(
            "upload_vcsr_mc_device: format arrays differ in length from the sizes they imply");
    if (!g_handle) check(vcsrmc_create(&g_handle), "upload_vcsr_mc_device");
    check(vcsrmc_upload(g_handle, V.M, V.N, V.segw, V.bundle, V.num_segments,
                        (int)V.group_depth.size(), (long long)V.val.size(),
                        (int)V.item_gbeg.size(), V.group_ptr.data(), V.group_depth.data(),
                        V.group_seg_base.data(), V.group_rows.data(), V.lcol.data(), V.val.data(),
                        V.item_gbeg.data(), V.item_gend.data(), V.scale, V.fp32 ? 1 : 0, nullptr),
          "upload_vcsr_mc_device");
    g_uploaded = true;
}

void run_vcsr_mc_spmm_gpu(const VCSRMC& V, const float* dB, int O, int tileK, float* dC,
                          hipStream_t st, float& ms) {
    if (V.item_gbeg.empty()) { ms = 0; return; }
    if (!g_uploaded) upload_vcsr_mc_device(V);
    const int status = vcsrmc_spmm(g_handle, dB, VCSRMC_B_F32, O, tileK, dC, st, &ms);
    if (status == VCSRMC_ERR_TILEK)
        throw std::runtime_error("vcsr_mc supports tileK in {16, 32, 64, 128}");
    check(status, "run_vcsr_mc_spmm_gpu");
}

void destroy_vcsr_mc_device(hipStream_t) {
    if (g_handle) check(vcsrmc_destroy(g_handle), "destroy_vcsr_mc_device");
    g_handle = nullptr;
    g_uploaded = false;
}

std::vector<int> rcm_column_order(const CSR& csr) {
    Dev<int> rp(csr.row_ptr), ci(csr.col);
    Dev<int> pos((size_t)csr.N);
    check(vcsrmc_rcm_order(rp.p, ci.p, csr.M, csr.N, csr.nnz, pos.p, nullptr), "rcm_column_order");
    std::vector<int> position((size_t)csr.N);
    pos.to_host(position);
    return position;
}

void apply_column_permutation(CSR& csr, std::vector<float>& hB, int O,
                              const std::vector<int>& position) {
    if ((int)position.size() != csr.N)
        throw std::runtime_error("apply_column_permutation: position must hold N entries");
    if (!hB.empty() && hB.size() != (size_t)csr.N * (size_t)O)
        throw std::runtime_error("apply_column_permutation: B must hold N x O values");
    Dev<int> rp(csr.row_ptr), ci(csr.col), pos(position);
    Dev<float> vv(csr.val);
    if (hB.empty()) {
        check(vcsrmc_apply_column_permutation(rp.p, ci.p, vv.p, csr.M, csr.N, csr.nnz, pos.p,
                                              nullptr, O, nullptr, nullptr),
              "apply_column_permutation");
    } else {
        Dev<float> b(hB), bout(hB.size());
        check(vcsrmc_apply_column_permutation(rp.p, ci.p, vv.p, csr.M, csr.N, csr.nnz, pos.p,
                                              b.p, O, bout.p, nullptr),
              "apply_column_permutation");
        bout.to_host(hB);
    }
    ci.to_host(csr.col);
    vv.to_host(csr.val);
}
