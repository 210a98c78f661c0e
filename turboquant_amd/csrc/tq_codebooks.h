// tq_codebooks.h -- core codec codebook tables (host side).
#pragma once

namespace tqh {
// Centroids (2^bits) and boundaries (2^bits - 1) for a table dimension;
// false for a dimension or bit width without a table.
bool core_codebook(int bits, int dim, const double **c, const double **b, int *nc);
}  // namespace tqh
