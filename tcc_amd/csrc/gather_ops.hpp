// Row- and column-scaled forms of the BCSR gathers and the TF32 pack
// (bcsr_spmm.hip), for products A X with A = diag(rowScale) * B *
// diag(colScale) over a pattern (or valued) B: X's rows are scaled while
// they are packed, and each output row's sum is scaled before it is stored
// or added.  The C-ABI entry points are these with null scales.  They set
// the library's last error and return its codes like the entry points.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/tcc_spmm_cnic.h"

namespace tcc {

// Rows of the slice maxima tf32_pack_scaled gathers (its atomics spread over
// them) and the most slices it takes (their maxima sit in LDS).
constexpr std::uint32_t kPackSliceMaxRows = 64;
constexpr std::uint32_t kPackMaxSlices = 16384;

// tcc_bcsr_spmm; rowScale (nullptr: none) has 8 entries per output window.
// rowLimit (0: none) is the number of rows of a Y that ends inside the last
// window (8 * num_rowWindows - 8 < rowLimit <= 8 * num_rowWindows), for
// adding (accumulate != 0) into a Y of exactly the matrix's rows; an
// ordinary (unphased) BCSR then neither reads nor writes rows past it.
int bcsr_spmm_scaled(const tcc_bcsr* A, const float* X, float* Y, std::uint32_t featureDim, int accumulate,
                     const float* rowScale, hipStream_t st, std::uint32_t rowLimit = 0);

// tcc_tf32_pack of colScale[r] * X[r] (colScale nullptr: X itself).  With
// sliceMax, the largest finite magnitude's bits of each slice of
// sliceWidth features (a multiple of 4) over all rows, in
// sliceMax[k * slices + s]: the maximum over k < kPackSliceMaxRows (slices
// at most kPackMaxSlices; the kPackSliceMaxRows * slices words are zeroed
// first).
int tf32_pack_scaled(const float* X, std::uint32_t rows, std::uint32_t featureDim, const float* colScale,
                     void* packed, hipStream_t st, std::uint32_t* sliceMax = nullptr, std::uint32_t sliceWidth = 0,
                     std::uint32_t slices = 0);

// tcc_bcsr_spmm_packed; rowScale and rowLimit as bcsr_spmm_scaled.
int bcsr_spmm_packed_scaled(const tcc_bcsr* A, const void* packedX, float* Y, std::uint32_t featureDim,
                            int accumulate, const float* rowScale, hipStream_t st, std::uint32_t rowLimit = 0);

}  // namespace tcc
