// csr.hpp -- the CSR container the VCSR-MC path takes as input, and its construction from
// Matrix Market coordinates.
//
// Same members, types and order as the reference's struct CSR (MuuSeoTia/VCSR_MC
// include/csr.hpp:8-13), and the same coo_to_csr (include/csr.hpp:16-42: rows bucketed, columns
// sorted within each row, values following, errors with the same texts), so existing callers
// compile unchanged.  Invariants the GPU format builder checks: row_ptr is monotone from 0 to
// nnz, and the columns of each row are strictly increasing (sorted, no duplicate coordinates).
#pragma once
#include <stdexcept>
#include <vector>

#include "mmio.hpp"

struct CSR {
    int M{0}, N{0}, nnz{0};
    std::vector<int> row_ptr;  // M + 1 offsets
    std::vector<int> col;      // nnz column indices
    std::vector<float> val;    // nnz values
};

// Entries ordered by (row, column) with two stable counting passes, columns first, then rows;
// an entry whose row or column lies outside the matrix, or two entries on one coordinate, are
// rejected.  All row indices are checked before any column index, as the reference does.
inline CSR coo_to_csr(const COO& coo) {
    const size_t n = coo.vals.size();
    if (coo.rows.size() != n || coo.cols.size() != n)
        throw std::runtime_error("COO arrays differ in length");
    CSR csr;
    csr.M = coo.M;
    csr.N = coo.N;
    csr.nnz = (int)n;
    for (int r : coo.rows)
        if (r < 0 || r >= coo.M) throw std::runtime_error("row idx out of range");
    for (int c : coo.cols)
        if (c < 0 || c >= coo.N) throw std::runtime_error("column idx out of range");

    // pass 1: entry order by column
    std::vector<int> cstart((size_t)coo.N + 1, 0);
    for (int c : coo.cols) ++cstart[(size_t)c + 1];
    for (int c = 0; c < coo.N; ++c) cstart[(size_t)c + 1] += cstart[c];
    std::vector<int> by_col(n);
    for (size_t i = 0; i < n; ++i) by_col[(size_t)cstart[coo.cols[i]]++] = (int)i;

    // pass 2: stable by row, so each row's entries come out in column order
    csr.row_ptr.assign((size_t)coo.M + 1, 0);
    for (int r : coo.rows) ++csr.row_ptr[(size_t)r + 1];
    for (int r = 0; r < coo.M; ++r) csr.row_ptr[(size_t)r + 1] += csr.row_ptr[r];
    std::vector<int> next(csr.row_ptr.begin(), csr.row_ptr.end() - 1);
    csr.col.resize(n);
    csr.val.resize(n);
    for (int i : by_col) {
        const int dst = next[coo.rows[i]]++;
        csr.col[dst] = coo.cols[i];
        csr.val[dst] = coo.vals[i];
    }
    for (int r = 0; r < coo.M; ++r)
        for (int p = csr.row_ptr[r] + 1; p < csr.row_ptr[(size_t)r + 1]; ++p)
            if (csr.col[p] == csr.col[p - 1])
                throw std::runtime_error(
                    "Duplicate MTX coordinates are unsupported; coalesce them before "
                    "benchmarking");
    return csr;
}
