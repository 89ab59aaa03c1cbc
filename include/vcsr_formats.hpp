// vcsr_formats.hpp -- drop-in C++ surface of the VCSR-MC SpMM path, backed by libvcsrmc.so.
//
// Declarations match MuuSeoTia/VCSR_MC include/vcsr_formats.hpp:11-26 (same names, argument
// meaning, struct members and error behaviour), so a caller such as the reference's driver
// (src/main.cpp:345-362) links against this library without source changes:
//   - invalid segw / tileK throw std::runtime_error (src/vcsr_mc.cu:26-27, 385-388);
//   - HIP runtime failures print a message and exit(EXIT_FAILURE) (include/cuda_check.hpp:7-14);
//   - one format at a time is held on the device; upload is a no-op once a format is
//     uploaded, destroy releases it (src/vcsr_mc.cu:126-131, 334, 403).
// Differences, both additive: csr_to_vcsr_mc runs on the GPU (its output arrays equal the
// reference's, with rows of equal count in a segment ordered by ascending row id), and a CSR
// whose rows are not strictly increasing is rejected with std::runtime_error.
// The C ABI underneath is include/vcsrmc.h.
#pragma once
#include <hip/hip_runtime.h>

#include <vector>

#include "csr.hpp"

// Factor A is divided by before the FP16 conversion (C is multiplied by it afterwards).
float half_scale(const CSR &csr);

struct VCSRMC {
    int M{0}, N{0}, segw{16}, bundle{16}, num_segments{0};
    std::vector<int> group_ptr, group_depth, group_seg_base, group_rows, lcol;
    std::vector<float> val;
    std::vector<int> item_gbeg, item_gend;  // groups [gbeg, gend) of one segment per item
    float scale{1.0f};
    bool fp32{false};  // vcsr_mc_fp32: FP32 operands and MFMA, scale = 1
};

VCSRMC csr_to_vcsr_mc(const CSR &csr, bool fp32 = false, int segw = 16);  // segw: 16, 32, 48, 64
void upload_vcsr_mc_device(const VCSRMC &V);
void run_vcsr_mc_spmm_gpu(const VCSRMC &V, const float *dB, int O, int tileK, float *dC,
                          hipStream_t st, float &ms);
void destroy_vcsr_mc_device(hipStream_t st);
