// COO -> BCSR / BCSC construction on gfx950.
//
// The reference's producer of these arrays (ipc_service, outside the
// repository) is absent; the layout here is the one its kernels consume
// (spmm_cnic/src/core/spmm_kernel.cu:87-121 for BCSR, :521-524, :600-615 and
// :689-690 for BCSC, :88-101 for the value order):
//   BCSR: per 8-row window, its distinct columns ascending, 8 per block.
//   BCSC: per 8-source window, its destination rows ordered by (degree desc,
//         dst asc), 8 per block — the SWTCF row order with one window per
//         super-window, so the SWTCF converter builds it.
// Both calls synchronise `stream` once to learn the block count, allocate the
// arrays in one hipMalloc (released with tcc_block_release) and return views.
#include <algorithm>
#include <cstring>
#include <vector>

#include "../../include/tcc_spmm_cnic.h"
#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "primitives.hpp"

namespace tcc {
namespace {

constexpr unsigned kThreads = 256;

inline unsigned ceil_log2(std::uint64_t x) {
    unsigned b = 0;
    while ((1ull << b) < x) ++b;
    return b;
}

inline std::size_t align_up(std::size_t x) { return (x + 255) & ~std::size_t(255); }

// Sort key (row window, column, row in window).  With phases > 1 the row
// window of an edge is phase(c) * windowsPerPhase + r / 8, where column c is
// in phase c * phases / numCols: the matrix is built as its column slices
// stacked vertically.
__global__ void bcsr_keys_kernel(const std::uint32_t* __restrict__ row, const std::uint32_t* __restrict__ col,
                                 std::uint32_t E, std::uint32_t numRows, std::uint32_t numCols, unsigned colBits,
                                 std::uint32_t phases, std::uint32_t windowsPerPhase,
                                 std::uint64_t* __restrict__ keys, std::uint32_t* __restrict__ perm,
                                 std::uint32_t* __restrict__ err) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    std::uint32_t r = row[e], c = col[e];
    if (r >= numRows || c >= numCols) {
        atomicMax(err, 1u);
        r = 0;
        c = 0;
    }
    const std::uint64_t phase = static_cast<std::uint64_t>(c) * phases / numCols;
    const std::uint64_t w = phase * windowsPerPhase + (r >> 3);
    keys[e] = ((w << colBits | c) << 3) | (r & 7u);
    perm[e] = e;
}

// Heads of (row window, column) runs; a repeated full key is a duplicate edge.
__global__ void bcsr_flags_kernel(const std::uint64_t* __restrict__ keys, std::uint32_t E, unsigned colBits,
                                  std::uint32_t* __restrict__ flags, std::uint32_t* __restrict__ rwCount,
                                  std::uint32_t* __restrict__ err) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint64_t k = keys[e];
    const bool head = e == 0 || (k >> 3) != (keys[e - 1] >> 3);
    if (e > 0 && k == keys[e - 1]) atomicMax(err, 2u);
    flags[e] = head ? 1u : 0u;
    if (head) aggregated_increment(rwCount, static_cast<std::uint32_t>(k >> (colBits + 3)));
}

__global__ void blocks_per_window_kernel(const std::uint32_t* __restrict__ cnt, std::uint32_t n,
                                         std::uint32_t* __restrict__ blocks) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) blocks[i] = (cnt[i] + 7) / 8;
}

// Column slots, bitmaps; remembers each edge's (block, bit) for the values.
__global__ void bcsr_place_kernel(const std::uint64_t* __restrict__ keys, std::uint32_t E, unsigned colBits,
                                  const std::uint32_t* __restrict__ flags, const std::uint32_t* __restrict__ pos,
                                  const std::uint32_t* __restrict__ rwFirst,
                                  const std::uint32_t* __restrict__ rowWindowOffset,
                                  std::uint32_t* __restrict__ sparseA2B,
                                  unsigned long long* __restrict__ tcLocalBit,
                                  std::uint64_t* __restrict__ edgeLoc) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint64_t k = keys[e];
    const std::uint32_t rw = static_cast<std::uint32_t>(k >> (colBits + 3));
    const std::uint32_t u = pos[e] + flags[e] - 1;  // distinct-column index
    const std::uint32_t kk = u - rwFirst[rw];
    const std::uint32_t blk = rowWindowOffset[rw] + kk / 8;
    const std::uint32_t c = kk & 7u;
    const std::uint32_t bit = static_cast<std::uint32_t>(k & 7u) * 8 + c;
    if (flags[e]) {
        const std::uint32_t colMask = colBits >= 32 ? 0xFFFFFFFFu : ((1u << colBits) - 1u);
        sparseA2B[static_cast<std::uint64_t>(blk) * 8 + c] = static_cast<std::uint32_t>(k >> 3) & colMask;
    }
    atomicOr(&tcLocalBit[blk], 1ull << bit);
    edgeLoc[e] = static_cast<std::uint64_t>(blk) * 64 + bit;
}

__global__ void popcount_kernel(const std::uint64_t* __restrict__ bits, std::uint32_t n,
                                std::uint32_t* __restrict__ out) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = static_cast<std::uint32_t>(__popcll(bits[i]));
}

// data[tcOffset[b] + rank of the entry's bit] = value of the edge.
__global__ void scatter_values_kernel(const std::uint64_t* __restrict__ edgeLoc,
                                      const std::uint32_t* __restrict__ perm, std::uint32_t E,
                                      const std::uint64_t* __restrict__ bits,
                                      const std::uint32_t* __restrict__ tcOffset, const float* __restrict__ val,
                                      float* __restrict__ data) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint64_t loc = edgeLoc[e];
    const std::uint64_t b = loc / 64;
    const unsigned bit = static_cast<unsigned>(loc % 64);
    const std::uint64_t below = bits[b] & ((1ull << bit) - 1ull);
    data[tcOffset[b] + __popcll(below)] = val ? val[perm[e]] : 1.0f;
}

// BCSC from SWTCF(S=1): global destination of each tile row.
__global__ void bcsc_rows_kernel(const std::uint32_t* __restrict__ colWindowOffset, std::uint32_t CW,
                                 const std::uint32_t* __restrict__ swRowOffset,
                                 const std::uint32_t* __restrict__ swRows, const std::uint32_t* __restrict__ tileRowSlot,
                                 std::uint32_t T, std::uint32_t* __restrict__ sparseA2C,
                                 std::uint32_t* __restrict__ slotToLoc) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= T * 8u) return;
    const std::uint32_t t = i / 8;
    std::uint32_t lo = 0, hi = CW;  // window of tile t: last w with colWindowOffset[w] <= t
    while (lo + 1 < hi) {
        const std::uint32_t mid = (lo + hi) / 2;
        if (colWindowOffset[mid] <= t) lo = mid; else hi = mid;
    }
    const std::uint32_t slot = tileRowSlot[i];
    if (slot == TCC_SWTCF_INVALID_ROW_SLOT) {
        sparseA2C[i] = TCC_SWTCF_INVALID_ROW_SLOT;
    } else {
        sparseA2C[i] = swRows[swRowOffset[lo] + slot];
        slotToLoc[swRowOffset[lo] + slot] = i;
    }
}

// Value placement for BCSC: edge (dst, src) -> tile row of dst in window src/8.
__global__ void bcsc_values_kernel(const std::uint32_t* __restrict__ dst, const std::uint32_t* __restrict__ src,
                                   const float* __restrict__ val, std::uint32_t E,
                                   const std::uint32_t* __restrict__ swRowOffset,
                                   const std::uint32_t* __restrict__ swRows,
                                   const std::uint32_t* __restrict__ slotToLoc,
                                   const std::uint64_t* __restrict__ bits, const std::uint32_t* __restrict__ tcOffset,
                                   float* __restrict__ data) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint32_t w = src[e] >> 3, c = src[e] & 7u, d = dst[e];
    std::uint32_t lo = swRowOffset[w], hi = swRowOffset[w + 1];
    while (lo < hi) {
        const std::uint32_t mid = (lo + hi) / 2;
        if (swRows[mid] < d) lo = mid + 1; else hi = mid;
    }
    const std::uint32_t loc = slotToLoc[lo];
    const std::uint32_t t = loc / 8, bit = (loc & 7u) * 8 + c;
    data[tcOffset[t] + __popcll(bits[t] & ((1ull << bit) - 1ull))] = val ? val[e] : 1.0f;
}

template <typename T>
struct DevBuf {
    T* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

}  // namespace
}  // namespace tcc

using namespace tcc;

extern "C" {

int tcc_block_release(void* allocation) {
    clear_last_error();
    if (allocation) TCC_HIP_CHECK(hipFree(allocation));
    return TCC_OK;
}

int tcc_coo_to_bcsr(const std::uint32_t* dRow, const std::uint32_t* dCol, const float* dVal, std::uint32_t nnz,
                    std::uint32_t numRows, std::uint32_t numCols, tcc_bcsr* out, void** allocation,
                    void* stream) {
    return tcc_coo_to_bcsr_phased(dRow, dCol, dVal, nnz, numRows, numCols, 1, out, allocation, stream);
}

int tcc_coo_to_bcsr_phased(const std::uint32_t* dRow, const std::uint32_t* dCol, const float* dVal,
                           std::uint32_t nnz, std::uint32_t numRows, std::uint32_t numCols, std::uint32_t phases,
                           tcc_bcsr* out, void** allocation, void* stream) {
    clear_last_error();
    TCC_REQUIRE(out && allocation && numRows >= 1 && numCols >= 1 && (nnz == 0 || (dRow && dCol)),
                TCC_ERR_INVALID_ARGUMENT, "invalid COO -> BCSR arguments");
    if (phases == 0) phases = 1;
    const hipStream_t st = as_stream(stream);
    const std::uint32_t windowsPerPhase = (numRows + 7) / 8;
    TCC_REQUIRE(static_cast<std::uint64_t>(windowsPerPhase) * phases < 0xFFFFFFFFull, TCC_ERR_UNSUPPORTED,
                "too many row windows for the phase count");
    const std::uint32_t E = nnz, RW = windowsPerPhase * phases;
    const unsigned colBits = std::max(1u, ceil_log2(numCols));
    TCC_REQUIRE(ceil_log2(RW) + colBits + 3 <= 64, TCC_ERR_UNSUPPORTED, "BCSR key exceeds 64 bits");
    std::memset(out, 0, sizeof(*out));
    *allocation = nullptr;

    // scratch: one allocation carved by the same function that sizes it
    const std::uint64_t En = std::max<std::uint32_t>(E, 1);
    const std::uint64_t tempElems =
        std::max({radix_temp_elems(En), scan_temp_elems(En + 1), scan_temp_elems(RW + 1)});
    std::uint64_t *keysA, *keysB, *edgeLoc;
    std::uint32_t *permA, *permB, *flags, *pos, *rwCount, *rwFirst, *rwBlocks, *temp, *small;
    auto carve = [&](char* base) {
        std::size_t off = 0;
        auto take = [&](std::size_t bytes) {
            char* p = base ? base + off : nullptr;
            off += align_up(bytes);
            return p;
        };
        keysA = reinterpret_cast<std::uint64_t*>(take(8 * En));
        keysB = reinterpret_cast<std::uint64_t*>(take(8 * En));
        permA = reinterpret_cast<std::uint32_t*>(take(4 * En));
        permB = reinterpret_cast<std::uint32_t*>(take(4 * En));
        flags = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        pos = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        edgeLoc = reinterpret_cast<std::uint64_t*>(take(8 * En));
        rwCount = reinterpret_cast<std::uint32_t*>(take(4 * (RW + 1)));
        rwFirst = reinterpret_cast<std::uint32_t*>(take(4 * (RW + 1)));
        rwBlocks = reinterpret_cast<std::uint32_t*>(take(4 * (RW + 1)));
        temp = reinterpret_cast<std::uint32_t*>(take(4 * tempElems));
        small = reinterpret_cast<std::uint32_t*>(take(256));  // [0]=err [1]=distinct [2]=blocks
        return off;
    };
    const std::size_t scratchBytes = carve(nullptr);
    DevBuf<char> scratch;
    TCC_HIP_CHECK(hipMalloc(&scratch.p, scratchBytes));
    carve(scratch.p);

    TCC_HIP_CHECK(fill<std::uint32_t>(small, 64, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(rwCount, RW + 1, 0u, st));
    std::uint64_t* sorted = keysA;
    std::uint32_t* perm = permA;
    if (E > 0) {
        hipLaunchKernelGGL(bcsr_keys_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, dRow, dCol, E,
                           numRows, numCols, colBits, phases, windowsPerPhase, keysA, permA, small);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(radix_sort_pairs(keysA, keysB, permA, permB, E, ceil_log2(RW) + colBits + 3, temp, &sorted,
                                       &perm, st));
        hipLaunchKernelGGL(bcsr_flags_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, E,
                           colBits, flags, rwCount, small);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(flags, pos, E, small + 1, temp, st));
    }
    TCC_HIP_CHECK(exclusive_scan(rwCount, rwFirst, RW, nullptr, temp, st));
    hipLaunchKernelGGL(blocks_per_window_kernel, dim3(grid_for(RW, kThreads)), dim3(kThreads), 0, st, rwCount,
                       RW, rwBlocks);
    TCC_LAUNCH_CHECK();

    std::uint32_t hostSmall[4] = {0, 0, 0, 0};
    // rowWindowOffset is computed straight into the output below; first learn B.
    TCC_HIP_CHECK(exclusive_scan(rwBlocks, rwBlocks, RW, small + 2, temp, st));
    TCC_HIP_CHECK(hipMemcpyAsync(hostSmall, small, sizeof(hostSmall), hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    if (hostSmall[0] != 0) {
        set_last_error(hostSmall[0] == 2 ? "duplicate (row, col) entries in the COO input"
                                         : "COO index out of range");
        return TCC_ERR_INVALID_ARGUMENT;
    }
    const std::uint32_t B = hostSmall[2];

    // outputs: rowWindowOffset[RW+1] tcOffset[B+1] sparseA2B[8B] tcLocalBit[B] data[E]
    const std::size_t outBytes = align_up(4 * (RW + 1)) + align_up(4 * (B + 1)) + align_up(32 * std::max(B, 1u)) +
                                 align_up(8 * std::max(B, 1u)) + align_up(4 * En);
    char* o = nullptr;
    TCC_HIP_CHECK(hipMalloc(&o, outBytes));
    char* q = o;
    auto takeOut = [&](std::size_t bytes) {
        char* p = q;
        q += align_up(bytes);
        return p;
    };
    auto* rowWindowOffset = reinterpret_cast<std::uint32_t*>(takeOut(4 * (RW + 1)));
    auto* tcOffset = reinterpret_cast<std::uint32_t*>(takeOut(4 * (B + 1)));
    auto* sparseA2B = reinterpret_cast<std::uint32_t*>(takeOut(32 * std::max(B, 1u)));
    auto* tcLocalBit = reinterpret_cast<std::uint64_t*>(takeOut(8 * std::max(B, 1u)));
    auto* data = reinterpret_cast<float*>(takeOut(4 * En));
    auto fail = [&](int rc) {
        (void)hipFree(o);
        return rc;
    };
    if (hipMemcpyAsync(rowWindowOffset, rwBlocks, 4 * RW, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        hipMemcpyAsync(rowWindowOffset + RW, small + 2, 4, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        fill<std::uint32_t>(sparseA2B, 8ull * B, TCC_SWTCF_INVALID_ROW_SLOT, st) != hipSuccess ||
        fill<std::uint64_t>(tcLocalBit, B, 0ull, st) != hipSuccess) {
        set_last_error("HIP error while initialising BCSR arrays");
        return fail(TCC_ERR_HIP);
    }
    if (E > 0) {
        hipLaunchKernelGGL(bcsr_place_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, E,
                           colBits, flags, pos, rwFirst, rowWindowOffset, sparseA2B,
                           reinterpret_cast<unsigned long long*>(tcLocalBit), edgeLoc);
        hipLaunchKernelGGL(popcount_kernel, dim3(grid_for(B, kThreads)), dim3(kThreads), 0, st, tcLocalBit, B,
                           flags);
        if (exclusive_scan(flags, tcOffset, B, tcOffset + B, temp, st) != hipSuccess) return fail(TCC_ERR_HIP);
        hipLaunchKernelGGL(scatter_values_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, edgeLoc,
                           perm, E, tcLocalBit, tcOffset, dVal, data);
    } else {
        (void)fill<std::uint32_t>(tcOffset, 1, 0u, st);
    }
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        set_last_error("HIP error while building BCSR");
        return fail(TCC_ERR_HIP);
    }
    out->num_rows = numRows;
    out->num_cols = numCols;
    out->nnz = E;
    out->num_TCBlocks = B;
    out->num_rowWindows = RW;
    out->rowWindowOffset = rowWindowOffset;
    out->tcOffset = tcOffset;
    out->sparseA2B = sparseA2B;
    out->tcLocalBit = tcLocalBit;
    out->data = dVal ? data : nullptr;
    out->phases = phases;
    *allocation = o;
    return TCC_OK;
}

int tcc_coo_to_bcsc(const std::uint32_t* dRow, const std::uint32_t* dCol, const float* dVal, std::uint32_t nnz,
                    std::uint32_t numRows, std::uint32_t numCols, tcc_bcsc* out, void** allocation,
                    void* stream) {
    clear_last_error();
    TCC_REQUIRE(out && allocation && numRows >= 1 && numCols >= 1 && (nnz == 0 || (dRow && dCol)),
                TCC_ERR_INVALID_ARGUMENT, "invalid COO -> BCSC arguments");
    const hipStream_t st = as_stream(stream);
    std::memset(out, 0, sizeof(*out));
    *allocation = nullptr;
    if (nnz == 0) {
        // every column window empty and no blocks, as tcc_coo_to_bcsr gives
        // for no edges (the converter below needs at least one edge)
        const std::uint32_t CW = (numCols + 7) / 8;
        const std::size_t offBytes = align_up(4ull * (CW + 1));
        char* o = nullptr;
        TCC_HIP_CHECK(hipMalloc(&o, offBytes + align_up(4) + align_up(32) + align_up(8)));
        if (fill<std::uint32_t>(reinterpret_cast<std::uint32_t*>(o), (offBytes + align_up(4) + align_up(32) + align_up(8)) / 4,
                                0u, st) != hipSuccess ||
            hipStreamSynchronize(st) != hipSuccess) {
            (void)hipFree(o);
            set_last_error("HIP error while building an empty BCSC");
            return TCC_ERR_HIP;
        }
        out->num_rows = numRows;
        out->num_cols = numCols;
        out->num_colWindows = CW;
        out->colWindowOffset = reinterpret_cast<std::uint32_t*>(o);
        out->tcOffset = reinterpret_cast<std::uint32_t*>(o + offBytes);
        out->sparseA2C = reinterpret_cast<std::uint32_t*>(o + offBytes + align_up(4));
        out->tcLocalBit = reinterpret_cast<std::uint64_t*>(o + offBytes + align_up(4) + align_up(32));
        *allocation = o;
        return TCC_OK;
    }
    tcc_swtcf_matrix m;
    tcc_swtcf_workspace ws;
    int rc = tcc_swtcf_alloc_matrix(&m, numRows, numCols, nnz, 1);
    if (rc) return rc;
    rc = tcc_swtcf_alloc_workspace(&ws, nnz, numCols, 1);
    if (rc) {
        tcc_swtcf_free_matrix(&m);
        return rc;
    }
    struct Cleanup {
        tcc_swtcf_matrix* m;
        tcc_swtcf_workspace* ws;
        ~Cleanup() {
            tcc_swtcf_free_workspace(ws);
            tcc_swtcf_free_matrix(m);
        }
    } cleanup{&m, &ws};
    rc = tcc_swtcf_convert(dRow, dCol, nnz, &m, &ws, stream);
    if (rc) return rc;
    const std::uint32_t CW = m.numColWindows;
    std::uint32_t hostErr = 0, T = 0, U = 0;
    TCC_HIP_CHECK(hipMemcpyAsync(&hostErr, ws.deviceError, 4, hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipMemcpyAsync(&T, m.colWindowOffset + CW, 4, hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipMemcpyAsync(&U, m.superWindowRowOffset + CW, 4, hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    TCC_REQUIRE(hostErr == 0, TCC_ERR_INVALID_ARGUMENT,
                "COO -> BCSC: converter error " + std::to_string(hostErr) + " (duplicates or indices out of range)");

    const std::size_t outBytes = align_up(4 * (CW + 1)) + align_up(4 * (T + 1)) + align_up(32 * std::max(T, 1u)) +
                                 align_up(8 * std::max(T, 1u)) + align_up(4 * nnz) + align_up(4 * std::max(U, 1u)) +
                                 align_up(4 * std::max(T, 1u)) + align_up(4 * scan_temp_elems(T + 1));
    char* o = nullptr;
    TCC_HIP_CHECK(hipMalloc(&o, outBytes));
    char* q = o;
    auto takeOut = [&](std::size_t bytes) {
        char* p = q;
        q += align_up(bytes);
        return p;
    };
    auto* colWindowOffset = reinterpret_cast<std::uint32_t*>(takeOut(4 * (CW + 1)));
    auto* tcOffset = reinterpret_cast<std::uint32_t*>(takeOut(4 * (T + 1)));
    auto* sparseA2C = reinterpret_cast<std::uint32_t*>(takeOut(32 * std::max(T, 1u)));
    auto* tcLocalBit = reinterpret_cast<std::uint64_t*>(takeOut(8 * std::max(T, 1u)));
    auto* data = reinterpret_cast<float*>(takeOut(4 * nnz));
    auto* slotToLoc = reinterpret_cast<std::uint32_t*>(takeOut(4 * std::max(U, 1u)));  // scratch tail
    auto* counts = reinterpret_cast<std::uint32_t*>(takeOut(4 * std::max(T, 1u)));
    auto* temp = reinterpret_cast<std::uint32_t*>(takeOut(4 * scan_temp_elems(T + 1)));
    auto fail = [&](int code) {
        (void)hipFree(o);
        return code;
    };
    if (hipMemcpyAsync(colWindowOffset, m.colWindowOffset, 4 * (CW + 1), hipMemcpyDeviceToDevice, st) !=
            hipSuccess ||
        hipMemcpyAsync(tcLocalBit, m.tileLocalBit, 8ull * T, hipMemcpyDeviceToDevice, st) != hipSuccess) {
        set_last_error("HIP copy failed while building BCSC");
        return fail(TCC_ERR_HIP);
    }
    if (T > 0) {
        hipLaunchKernelGGL(bcsc_rows_kernel, dim3(grid_for(8ull * T, kThreads)), dim3(kThreads), 0, st,
                           m.colWindowOffset, CW, m.superWindowRowOffset, m.superWindowRows, m.tileRowSlot, T,
                           sparseA2C, slotToLoc);
        hipLaunchKernelGGL(popcount_kernel, dim3(grid_for(T, kThreads)), dim3(kThreads), 0, st, tcLocalBit, T,
                           counts);
    }
    if (exclusive_scan(counts, tcOffset, T, tcOffset + T, temp, st) != hipSuccess) return fail(TCC_ERR_HIP);
    hipLaunchKernelGGL(bcsc_values_kernel, dim3(grid_for(nnz, kThreads)), dim3(kThreads), 0, st, dRow, dCol, dVal,
                       nnz, m.superWindowRowOffset, m.superWindowRows, slotToLoc, tcLocalBit, tcOffset, data);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        set_last_error("HIP error while building BCSC");
        return fail(TCC_ERR_HIP);
    }
    out->num_rows = numRows;
    out->num_cols = numCols;
    out->nnz = nnz;
    out->num_TCBlocks = T;
    out->num_colWindows = CW;
    out->colWindowOffset = colWindowOffset;
    out->tcOffset = tcOffset;
    out->sparseA2C = sparseA2C;
    out->tcLocalBit = tcLocalBit;
    out->data = dVal ? data : nullptr;
    *allocation = o;
    return TCC_OK;
}

}  // extern "C"
