// tcc_swtcf.hpp — the reference's C++ converter / SpMM API on top of the
// C-ABI of libtcc_swtcf.so (include/tcc_swtcf.h), for MI355X (gfx950).
//
// Same names, argument order and defaults as the reference headers, with
// cudaStream_t -> hipStream_t:
//   types      include/types.h:7-10
//   constants  include/swtcf_convert.cuh:7-11, include/swtcf_spmm.cuh:7-8
//   structs    include/swtcf_convert.cuh:13-72
//   functions  include/swtcf_convert.cuh:74-78, include/swtcf_spmm.cuh:10-25
// Errors throw std::runtime_error carrying tcc_last_error(), as the
// reference does for invalid sizes and API failures
// (src/swtcf_convert.cu:24-33, :1120-1130, :1312-1333, :1762-1777).
// Asynchronous device errors are reported through workspace.deviceError
// (codes 1-4 as the reference, 5 = src >= cols, 6 = dst >= rows), read by the
// caller after a sync.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "tcc_swtcf.h"

using IndexType = std::uint32_t;
using OffsetType = std::uint32_t;
using ValueType = float;
using BitmapType = std::uint64_t;

constexpr IndexType SWTCF_COL_WINDOW_WIDTH = TCC_SWTCF_COL_WINDOW_WIDTH;
constexpr IndexType SWTCF_TILE_ROWS = TCC_SWTCF_TILE_ROWS;
constexpr IndexType SWTCF_REPEAT_CACHE_SIZE = TCC_SWTCF_REPEAT_CACHE_SIZE;
constexpr IndexType SWTCF_MAX_SUPER_WINDOW_SIZE = TCC_SWTCF_MAX_SUPER_WINDOW_SIZE;
constexpr std::uint8_t SWTCF_INVALID_CACHE_SLOT = TCC_SWTCF_INVALID_CACHE_SLOT;
constexpr IndexType SWTCF_FEATURE_DIM = TCC_SWTCF_FEATURE_DIM;
constexpr IndexType SWTCF_DEFAULT_TC_THRESHOLD = TCC_SWTCF_DEFAULT_TC_THRESHOLD;

// The device SWTCF matrix: the C struct's fields and order, default values
// of the reference (colWindowWidth = tileRows = 8, everything else 0/null).
struct DeviceSWTCFMatrix : tcc_swtcf_matrix {
    DeviceSWTCFMatrix() : tcc_swtcf_matrix{} {
        colWindowWidth = SWTCF_COL_WINDOW_WIDTH;
        tileRows = SWTCF_TILE_ROWS;
    }
};

// Converter workspace.  Its scratch layout is this library's (one device
// allocation, no hash table); deviceNumGroups and deviceError keep the
// reference's meaning (swtcf_convert_main.cu:419-428).
struct SWTCFConvertWorkspace : tcc_swtcf_workspace {
    SWTCFConvertWorkspace() : tcc_swtcf_workspace{} {}
};

namespace tcc_detail {
inline void check(int rc, const char* what) {
    if (rc != 0) throw std::runtime_error(std::string(what) + ": " + tcc_last_error());
}
}  // namespace tcc_detail

inline void allocateDeviceSWTCF(DeviceSWTCFMatrix& matrix, IndexType rows, IndexType cols, IndexType nnz,
                                IndexType superWindowSize) {
    tcc_detail::check(tcc_swtcf_alloc_matrix(&matrix, rows, cols, nnz, superWindowSize), "allocateDeviceSWTCF");
}

inline void freeDeviceSWTCF(DeviceSWTCFMatrix& matrix) {
    tcc_detail::check(tcc_swtcf_free_matrix(&matrix), "freeDeviceSWTCF");
    matrix.colWindowWidth = SWTCF_COL_WINDOW_WIDTH;
    matrix.tileRows = SWTCF_TILE_ROWS;
}

inline void allocateSWTCFConvertWorkspace(SWTCFConvertWorkspace& workspace, IndexType edgeCapacity, IndexType numSrc,
                                          IndexType superWindowSize) {
    tcc_detail::check(tcc_swtcf_alloc_workspace(&workspace, edgeCapacity, numSrc, superWindowSize),
                      "allocateSWTCFConvertWorkspace");
}

inline void freeSWTCFConvertWorkspace(SWTCFConvertWorkspace& workspace) {
    tcc_detail::check(tcc_swtcf_free_workspace(&workspace), "freeSWTCFConvertWorkspace");
}

inline void convertCOOToSWTCF(const IndexType* deviceDst, const IndexType* deviceSrc, IndexType numEdges,
                              DeviceSWTCFMatrix& output, SWTCFConvertWorkspace& workspace, hipStream_t stream = 0) {
    tcc_detail::check(tcc_swtcf_convert(deviceDst, deviceSrc, numEdges, &output, &workspace, stream),
                      "convertCOOToSWTCF");
}

inline void launchSWTCFSpMM(const DeviceSWTCFMatrix& matrix, const ValueType* matrixX, ValueType* matrixY,
                            IndexType tcThreshold = SWTCF_DEFAULT_TC_THRESHOLD, hipStream_t stream = 0) {
    tcc_detail::check(tcc_swtcf_spmm(&matrix, matrixX, matrixY, tcThreshold, stream), "launchSWTCFSpMM");
}

inline void launchSWTCFSpMMQuantized(const DeviceSWTCFMatrix& matrix, const std::int8_t* quantizedX,
                                     const ValueType* scales, const IndexType* srcGlobal, ValueType* matrixY,
                                     IndexType tcThreshold = SWTCF_DEFAULT_TC_THRESHOLD, hipStream_t stream = 0) {
    tcc_detail::check(tcc_swtcf_spmm_quantized(&matrix, quantizedX, scales, srcGlobal, matrixY, tcThreshold, stream),
                      "launchSWTCFSpMMQuantized");
}
