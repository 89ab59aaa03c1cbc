// cuda_check.hpp -- the HIP error check the reference's host code uses (MuuSeoTia/VCSR_MC
// include/cuda_check.hpp:7-14): a failing runtime call prints where it failed and what the
// runtime said, then ends the process with EXIT_FAILURE.  The reference's kernel-file helper
// check_shared_memory (:16-29) belongs to its own multiply kernels, which libvcsrmc.so replaces,
// and is not part of this surface.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

inline void vcsrmc_hip_check_or_exit(hipError_t status, const char* call, const char* file,
                                     int line) {
    if (status == hipSuccess) return;
    std::fprintf(stderr, "HIP error %s:%d: %s: %s\n", file, line, call,
                 hipGetErrorString(status));
    std::exit(EXIT_FAILURE);
}

#define CUDA_CHECK(call) vcsrmc_hip_check_or_exit((call), #call, __FILE__, __LINE__)
