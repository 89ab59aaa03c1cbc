// ref_harness.cpp -- C entry points over the reference's own host format builder.
//
// TEST INFRASTRUCTURE ONLY.  oracle/Makefile compiles MuuSeoTia/VCSR_MC's src/vcsr_mc.cu
// where it lies (with the reference's own HIP flags, CMakeLists.txt:24-27) and links it with
// this file into oracle/_ref/libvcsrmc_ref.so.  Tests call it on the CPU to pin the oracle's
// restatement of csr_to_vcsr_mc (src/vcsr_mc.cu:25-123), half_scale (src/vcsr_mc.cu:14-22)
// and the column reordering (include/reorder.hpp, a header-only part of the reference), and
// to write the golden fixtures under tests/golden/; GPU tests call ref_spmm_gpu to check the
// library's product against the reference's own kernels (src/vcsr_mc.cu:143-394) on the same
// inputs.
#include <cstdlib>
#include <cstring>
#include <exception>

#include <algorithm>

#include "vcsr_formats.hpp"   // the reference's header (include/vcsr_formats.hpp)
#include "reorder.hpp"        // the reference's header (include/reorder.hpp)
#include "../oracle/vcsrmc_oracle.h"

namespace {
template <typename T>
T* dup(const std::vector<T>& v) {
    T* p = static_cast<T*>(std::malloc(sizeof(T) * (v.size() ? v.size() : 1)));
    if (p && !v.empty()) std::memcpy(p, v.data(), sizeof(T) * v.size());
    return p;
}
}  // namespace

extern "C" {

// Runs the reference's csr_to_vcsr_mc on a host CSR.  Returns 0, or 1 when the reference
// threw (its message is copied into err).  The arrays are malloc'd; free with orc_free.
int ref_build(const int* row_ptr, const int* col, const float* val, int M, int N, int segw,
              int fp32, orc_format* out, char* err, int errlen) {
    std::memset(out, 0, sizeof *out);
    try {
        CSR csr;
        csr.M = M; csr.N = N; csr.nnz = M ? row_ptr[M] : 0;
        csr.row_ptr.assign(row_ptr, row_ptr + M + 1);
        csr.col.assign(col, col + csr.nnz);
        csr.val.assign(val, val + csr.nnz);
        VCSRMC V = csr_to_vcsr_mc(csr, fp32 != 0, segw);
        out->M = V.M; out->N = V.N; out->segw = V.segw; out->bundle = V.bundle;
        out->num_segments = V.num_segments;
        out->G = (int)V.group_depth.size();
        out->nval = (long long)V.val.size();
        out->nitems = (int)V.item_gbeg.size();
        out->group_ptr = dup(V.group_ptr);
        out->group_depth = dup(V.group_depth);
        out->group_seg_base = dup(V.group_seg_base);
        out->group_rows = dup(V.group_rows);
        out->lcol = dup(V.lcol);
        out->val = dup(V.val);
        out->item_gbeg = dup(V.item_gbeg);
        out->item_gend = dup(V.item_gend);
        out->scale = V.scale;
        out->fp32 = V.fp32 ? 1 : 0;
        return 0;
    } catch (const std::exception& e) {
        if (err && errlen > 0) { std::strncpy(err, e.what(), errlen - 1); err[errlen - 1] = 0; }
        return 1;
    }
}

// C = A.B by the reference's own path on the current GPU: csr_to_vcsr_mc, then
// upload_vcsr_mc_device and run_vcsr_mc_spmm_gpu (src/vcsr_mc.cu:332-394; its kernels
// vcsr_mc / vcsr_mc_fp32 accumulate into C with atomicAdd), then destroy_vcsr_mc_device.  dB
// (N x O floats) and dC (M x O floats, accumulated into) are device pointers.  Returns 0, or 1
// when the reference threw (message in err).
int ref_spmm_gpu(const int* row_ptr, const int* col, const float* val, int M, int N, int segw,
                 int fp32, const float* dB, int O, int tileK, float* dC, char* err, int errlen) {
    try {
        CSR csr;
        csr.M = M; csr.N = N; csr.nnz = M ? row_ptr[M] : 0;
        csr.row_ptr.assign(row_ptr, row_ptr + M + 1);
        csr.col.assign(col, col + csr.nnz);
        csr.val.assign(val, val + csr.nnz);
        VCSRMC V = csr_to_vcsr_mc(csr, fp32 != 0, segw);
        destroy_vcsr_mc_device(nullptr);
        upload_vcsr_mc_device(V);
        float ms = 0.f;
        run_vcsr_mc_spmm_gpu(V, dB, O, tileK, dC, nullptr, ms);
        destroy_vcsr_mc_device(nullptr);
        return 0;
    } catch (const std::exception& e) {
        if (err && errlen > 0) { std::strncpy(err, e.what(), errlen - 1); err[errlen - 1] = 0; }
        return 1;
    }
}

float ref_half_scale(const float* val, int nnz) {
    CSR csr;
    csr.nnz = nnz;
    csr.val.assign(val, val + nnz);
    return half_scale(csr);
}

// std::sort with the reference's comparator shape (include/reorder.hpp:67-68), as compiled
// here: pins the oracle's restatement of its steps.
void ref_std_sort_by_key(int* a, long long n, const int* key) {
    std::sort(a, a + n, [&](int x, int y) { return key[x] < key[y]; });
}

// Keys that drive std::sort into its heapsort fallback: McIlroy's adversary ("A Killer
// Adversary for Quicksort", Software: Practice and Experience 29(4), 1999) answers the sort's
// comparisons lazily, freezing values so that every pivot is bad.  Running std::sort again on
// the frozen keys takes the same path.  keys[n] receives a permutation of 0..n-1.
void ref_sort_adversary(int n, int* keys) {
    std::vector<int> val(n), a(n);
    const int gas = n;
    int nsolid = 0, candidate = 0;
    for (int i = 0; i < n; ++i) { val[i] = gas; a[i] = i; }
    std::sort(a.begin(), a.end(), [&](int x, int y) {
        if (val[x] == gas && val[y] == gas) {
            if (x == candidate) val[x] = nsolid++;
            else val[y] = nsolid++;
        }
        if (val[x] == gas) candidate = x;
        else if (val[y] == gas) candidate = y;
        return val[x] < val[y];
    });
    for (int i = 0; i < n; ++i) {
        if (val[i] == gas) val[i] = nsolid++;
        keys[i] = val[i];
    }
}

// std::partial_sort(a, a + n, a + n) with the same comparator: the heapsort step std::sort
// falls back to.
void ref_partial_sort_by_key(int* a, long long n, const int* key) {
    std::partial_sort(a, a + n, a + n, [&](int x, int y) { return key[x] < key[y]; });
}

static CSR make_csr(const int* row_ptr, const int* col, const float* val, int M, int N) {
    CSR csr;
    csr.M = M; csr.N = N; csr.nnz = M ? row_ptr[M] : 0;
    csr.row_ptr.assign(row_ptr, row_ptr + M + 1);
    csr.col.assign(col, col + csr.nnz);
    if (val) csr.val.assign(val, val + csr.nnz);
    else csr.val.assign(csr.nnz, 1.0f);
    return csr;
}

// rcm_column_order (include/reorder.hpp:17-77): position[N].
void ref_rcm_order(const int* row_ptr, const int* col, int M, int N, int* position) {
    const std::vector<int> pos = rcm_column_order(make_csr(row_ptr, col, nullptr, M, N));
    std::copy(pos.begin(), pos.end(), position);
}

// apply_column_permutation (include/reorder.hpp:82-108): col/val relabelled in place,
// B (N x O) permuted in place.
void ref_apply_column_permutation(const int* row_ptr, int* col, float* val, int M, int N,
                                  const int* position, float* B, int O) {
    CSR csr = make_csr(row_ptr, col, val, M, N);
    std::vector<float> hB;
    if (B) hB.assign(B, B + (size_t)N * O);
    apply_column_permutation(csr, hB, O, std::vector<int>(position, position + N));
    std::copy(csr.col.begin(), csr.col.end(), col);
    std::copy(csr.val.begin(), csr.val.end(), val);
    if (B) std::copy(hB.begin(), hB.end(), B);
}

}  // extern "C"
