// csr.hpp -- the CSR container the VCSR-MC path takes as input.
//
// Same members, types and order as the reference's struct CSR (MuuSeoTia/VCSR_MC
// include/csr.hpp:8-13) so existing callers compile unchanged.  Invariants the GPU format
// builder checks (the reference's coo_to_csr establishes them, include/csr.hpp:28-40):
// row_ptr is monotone from 0 to nnz, and the columns of each row are strictly increasing
// (sorted, no duplicate coordinates).
#pragma once
#include <vector>

struct CSR {
    int M{0}, N{0}, nnz{0};
    std::vector<int> row_ptr;  // M + 1 offsets
    std::vector<int> col;      // nnz column indices
    std::vector<float> val;    // nnz values
};
