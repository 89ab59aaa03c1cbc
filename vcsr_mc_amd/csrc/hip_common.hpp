// hip_common.hpp -- error plumbing and wave64 helpers shared by the VCSR-MC HIP sources.
// Target: gfx950 (CDNA4), 64-lane wavefronts.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

namespace vcsrmc {

// Internal error: carries a C-ABI status code; converted to a return value at the ABI.
struct Error : std::runtime_error {
    int status;
    Error(int s, const std::string& m) : std::runtime_error(m), status(s) {}
};

[[noreturn]] void throw_hip(hipError_t e, const char* what, const char* file, int line);

#define VCSRMC_HIP(call)                                                        \
    do {                                                                        \
        const hipError_t e_ = (call);                                           \
        if (e_ != hipSuccess) ::vcsrmc::throw_hip(e_, #call, __FILE__, __LINE__); \
    } while (0)

constexpr int kWave = 64;

// ---- device helpers -------------------------------------------------------------------

__device__ __forceinline__ int lane_id() { return (int)__lane_id(); }

struct OpAdd {
    template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
    template <typename T> __device__ __forceinline__ T operator()(T a, T b) const { return a > b ? a : b; }
};

// DPP row_shr:n (dpp_ctrl 0x110 + n) inside each row of 16 lanes; lanes whose source lies
// outside the row receive `identity` (the old value, bound_ctrl off).
__device__ __forceinline__ int shr_row(int x, int n, int identity) {
    switch (n) {
        case 1: return __builtin_amdgcn_update_dpp(identity, x, 0x111, 0xf, 0xf, false);
        case 2: return __builtin_amdgcn_update_dpp(identity, x, 0x112, 0xf, 0xf, false);
        case 4: return __builtin_amdgcn_update_dpp(identity, x, 0x114, 0xf, 0xf, false);
        default: return __builtin_amdgcn_update_dpp(identity, x, 0x118, 0xf, 0xf, false);
    }
}

// Inclusive prefix over the 64 lanes of a wave: four DPP row_shr steps scan each row of 16
// lanes, then v_readlane carries the row totals (lanes 15, 31, 47) into later rows.
template <typename Op>
__device__ __forceinline__ int wave_scan_i32(int x, Op op, int identity) {
    x = op(x, shr_row(x, 1, identity));
    x = op(x, shr_row(x, 2, identity));
    x = op(x, shr_row(x, 4, identity));
    x = op(x, shr_row(x, 8, identity));
    const int row = lane_id() >> 4;
    const int t15 = __builtin_amdgcn_readlane(x, 15);
    const int t31 = __builtin_amdgcn_readlane(x, 31);
    const int t47 = __builtin_amdgcn_readlane(x, 47);
    // t15, t31, t47 are the totals of rows 0, 1 and 2 on their own.
    int carry = identity;
    if (row >= 1) carry = t15;
    if (row >= 2) carry = op(t15, t31);
    if (row >= 3) carry = op(op(t15, t31), t47);
    return row ? op(carry, x) : x;
}

template <typename Op>
__device__ __forceinline__ long long wave_scan_i64(long long x, Op op, long long identity) {
    // 64-bit: Hillis-Steele with 32-bit DPP moves of both halves.
    auto shr64 = [&](long long v, int n) -> long long {
        const int lo = (int)(unsigned long long)v, hi = (int)((unsigned long long)v >> 32);
        const int ilo = (int)(unsigned long long)identity, ihi = (int)((unsigned long long)identity >> 32);
        const unsigned a = (unsigned)shr_row(lo, n, ilo), b = (unsigned)shr_row(hi, n, ihi);
        return (long long)(((unsigned long long)b << 32) | a);
    };
    x = op(x, shr64(x, 1));
    x = op(x, shr64(x, 2));
    x = op(x, shr64(x, 4));
    x = op(x, shr64(x, 8));
    auto rl = [](long long v, int l) -> long long {
        const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned long long)v, l);
        const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)((unsigned long long)v >> 32), l);
        return (long long)(((unsigned long long)hi << 32) | lo);
    };
    const int row = lane_id() >> 4;
    const long long t15 = rl(x, 15), t31 = rl(x, 31), t47 = rl(x, 47);
    long long carry = identity;
    if (row >= 1) carry = t15;
    if (row >= 2) carry = op(t15, t31);
    if (row >= 3) carry = op(op(t15, t31), t47);
    return row ? op(carry, x) : x;
}

template <typename T, typename Op>
__device__ __forceinline__ T wave_scan(T x, Op op, T identity) {
    if constexpr (sizeof(T) == 8) return (T)wave_scan_i64((long long)x, op, (long long)identity);
    else return (T)wave_scan_i32((int)x, op, (int)identity);
}

// Broadcast lane 63 (the inclusive total of a scan).
template <typename T>
__device__ __forceinline__ T wave_last(T x) {
    if constexpr (sizeof(T) == 8) {
        const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned long long)x, 63);
        const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)((unsigned long long)x >> 32), 63);
        return (T)(((unsigned long long)hi << 32) | lo);
    } else {
        return (T)__builtin_amdgcn_readlane((int)x, 63);
    }
}

inline int bits_for(unsigned long long v) {  // number of bits needed to hold values 0..v
    int b = 0;
    while (v) { ++b; v >>= 1; }
    return b;
}

inline unsigned grid_for(long long n, int per_block) {
    return (unsigned)((n + per_block - 1) / per_block);
}

}  // namespace vcsrmc
