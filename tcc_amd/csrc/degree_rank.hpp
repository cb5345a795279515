// Degree ranks of the rows or columns of a COO matrix, for the
// degree-sorted formats (row super-window BCSR, dense hub tiles): rank[i] is
// the position of index i when the indices are ordered by degree
// (descending) and then by index (ascending).
#pragma once

#include "common.hpp"
#include "primitives.hpp"

namespace tcc {
namespace {

__global__ void degree_kernel(const std::uint32_t* __restrict__ idx, std::uint32_t E, std::uint32_t limit,
                              std::uint32_t* __restrict__ deg, std::uint32_t* __restrict__ err) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint32_t v = idx[e];
    if (v >= limit) {
        atomicMax(err, 1u);
        return;
    }
    atomicAdd(&deg[v], 1u);
}

// key = (~deg << idBits) | id: ascending order = degree descending, ids ascending.
__global__ void degree_keys_kernel(const std::uint32_t* __restrict__ deg, std::uint32_t n, unsigned idBits,
                                   std::uint64_t* __restrict__ keys) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) keys[i] = (static_cast<std::uint64_t>(0xFFFFFFFFu - deg[i]) << idBits) | i;
}

// order[s] = id at sorted position s (0xFFFFFFFF for s in [n, padded)),
// rank[id] = s.  `order` may be null.
__global__ void order_rank_kernel(const std::uint64_t* __restrict__ sorted, std::uint32_t n, std::uint32_t padded,
                                  unsigned idBits, std::uint32_t* __restrict__ order, std::uint32_t* __restrict__ rank) {
    const std::uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= padded) return;
    if (s >= n) {
        if (order) order[s] = 0xFFFFFFFFu;
        return;
    }
    const std::uint32_t id = static_cast<std::uint32_t>(sorted[s] & ((1ull << idBits) - 1ull));
    if (order) order[s] = id;
    rank[id] = s;
}

inline unsigned rank_bits(std::uint64_t x) {
    unsigned b = 0;
    while ((1ull << b) < x) ++b;
    return b;
}

// deg[0..limit) += occurrences of each index in idx[0..E); indices >= limit
// set *err to 1.  deg must be zeroed by the caller.
inline hipError_t degree_histogram(const std::uint32_t* idx, std::uint32_t E, std::uint32_t limit,
                                   std::uint32_t* deg, std::uint32_t* err, hipStream_t st) {
    if (E == 0) return hipSuccess;
    hipLaunchKernelGGL(degree_kernel, dim3(grid_for(E, 256)), dim3(256), 0, st, idx, E, limit, deg, err);
    return hipGetLastError();
}

// rank[] and (optionally) order[] of n indices with degrees deg[]; keysA,
// keysB hold n u64 each, temp radix_temp_elems(n) u32.
inline hipError_t degree_ranks(const std::uint32_t* deg, std::uint32_t n, std::uint32_t padded, std::uint32_t* rank,
                               std::uint32_t* order, std::uint64_t* keysA, std::uint64_t* keysB, std::uint32_t* temp,
                               hipStream_t st) {
    const unsigned idBits = std::max(1u, rank_bits(n));
    hipLaunchKernelGGL(degree_keys_kernel, dim3(grid_for(n, 256)), dim3(256), 0, st, deg, n, idBits, keysA);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    std::uint64_t* sorted = nullptr;
    e = radix_sort(keysA, keysB, n, 32 + idBits, temp, &sorted, st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(order_rank_kernel, dim3(grid_for(padded, 256)), dim3(256), 0, st, sorted, n, padded, idBits,
                       order, rank);
    return hipGetLastError();
}

}  // namespace
}  // namespace tcc
