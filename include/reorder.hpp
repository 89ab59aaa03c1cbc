// reorder.hpp -- drop-in column reordering of the VCSR-MC path, computed on the GPU by
// libvcsrmc.so.
//
// Same two functions, names, arguments and results as MuuSeoTia/VCSR_MC include/reorder.hpp
// (there inline host code): rcm_column_order returns new_position[old_column] of the reverse
// Cuthill-McKee order of the symmetrised pattern, element for element the reference's, tie
// order included (reorder.hpp:17-77); apply_column_permutation relabels A's columns, keeps each
// row sorted, and permutes the rows of B to match, so C = (A P)(P^T B) = A B
// (reorder.hpp:82-108).  Errors: an invalid CSR or position throws std::runtime_error; HIP
// runtime failures print a message and exit(EXIT_FAILURE), as elsewhere in this surface.
// The C ABI underneath is vcsrmc_rcm_order / vcsrmc_apply_column_permutation (vcsrmc.h).
#pragma once
#include <vector>

#include "csr.hpp"

std::vector<int> rcm_column_order(const CSR &csr);
void apply_column_permutation(CSR &csr, std::vector<float> &hB, int O,
                              const std::vector<int> &position);
