// mtx_dump.cpp -- test infrastructure (never linked into the product): reads a Matrix Market
// file with whichever read_matrix_market_coo / coo_to_csr the include path provides and prints
// the CSR, or the error text:
//   OK M N nnz
//   row_ptr values, one line;  col values, one line;  val bit patterns (hex), one line
//   ERR <message>
// Built against the reference's headers (oracle/Makefile, _ref/mtx_ref_dump) it writes the
// reference's result for the committed fixtures; built against this repository's include/ it
// gives the drop-in header's result for the same files.
#include <cstdio>
#include <cstring>
#include <exception>
#include <string>

#include "csr.hpp"

int main(int argc, char** argv) {
    if (argc != 2) {
        std::fprintf(stderr, "usage: %s file.mtx\n", argv[0]);
        return 2;
    }
    try {
        const CSR a = coo_to_csr(read_matrix_market_coo(argv[1]));
        std::printf("OK %d %d %d\n", a.M, a.N, a.nnz);
        for (int x : a.row_ptr) std::printf("%d ", x);
        std::printf("\n");
        for (int x : a.col) std::printf("%d ", x);
        std::printf("\n");
        for (float v : a.val) {
            unsigned u;
            std::memcpy(&u, &v, 4);
            std::printf("%08x ", u);
        }
        std::printf("\n");
    } catch (const std::exception& e) {
        std::printf("ERR %s\n", e.what());
    }
    return 0;
}
