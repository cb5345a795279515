// COO -> SWTCF conversion on gfx950 (reference: src/swtcf_convert.cu).
//
// Design (deterministic, no hash table, no atomic ranks):
//   1. One stable LSD radix sort of a packed edge key
//        key = sw | dst | wi | lc     (sw = super-window, wi = window in sw,
//                                      lc = src & 7; high to low bits)
//      sized to the bits the matrix needs (a 233k x 233k graph with S = 16
//      needs 36 bits = 5 passes).
//   2. Run boundaries of key>>3 are the (window, dst) groups (degree = run
//      length, bitmap = OR of 1<<lc); runs of key>>(3+wiBits) are the
//      distinct (super-window, dst) rows, already in dst-ascending slot order,
//      and their run length in groups is the occurrence count.
//   3. Per super-window, one workgroup walks its groups in order and gives
//      each its rank inside its (window, degree) bucket with a stable
//      wave-ballot multisplit, which is exactly the canonical
//      (degree desc, dst asc) row order; then it ranks the repeated rows by
//      (occurrence desc, slot asc) for the repeat cache.
// Degree histograms use atomics only to count, which is order-independent.
#include <algorithm>
#include <cstring>
#include <new>

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

struct KeyLayout {
    unsigned wiBits, dstBits, swBits, total;
};

inline KeyLayout key_layout(std::uint32_t rows, std::uint32_t S, std::uint32_t numSuperWindows) {
    KeyLayout k;
    k.wiBits = ceil_log2(S);
    k.dstBits = rows ? std::max(1u, ceil_log2(rows)) : 32u;
    k.swBits = ceil_log2(numSuperWindows);
    k.total = k.swBits + k.dstBits + k.wiBits + 3;
    return k;
}

// Byte layout of the workspace scratch allocation.
struct Carve {
    std::uint64_t* keysA;
    std::uint64_t* keysB;
    std::uint32_t* flags;          // [E+1] group heads, then row heads
    std::uint32_t* pos;            // [E+1] exclusive scans of flags
    std::uint32_t* groupStart;     // [E+1]
    std::uint32_t* groupInfo;      // [E]   bits | degree << 8
    std::uint32_t* rowStartGroup;  // [E+1]
    std::uint32_t* wdCount;        // [CW*8]
    std::uint32_t* wdBase;         // [CW*8]
    std::uint32_t* wActive;        // [CW]
    std::uint32_t* wTiles;         // [CW]
    std::uint32_t* numRows;        // [1]
    std::uint32_t* temp;           // scan / sort scratch
    std::size_t bytes;
};

inline std::size_t align_up(std::size_t x) { return (x + 255) & ~std::size_t(255); }

inline Carve carve(char* base, std::uint64_t E, std::uint64_t CW, std::uint64_t SW) {
    Carve c{};
    std::size_t off = 0;
    auto take = [&](std::size_t bytes) {
        char* p = base ? base + off : nullptr;
        off = align_up(off + bytes);
        return p;
    };
    c.keysA = reinterpret_cast<std::uint64_t*>(take(8 * E));
    c.keysB = reinterpret_cast<std::uint64_t*>(take(8 * E));
    c.flags = reinterpret_cast<std::uint32_t*>(take(4 * (E + 1)));
    c.pos = reinterpret_cast<std::uint32_t*>(take(4 * (E + 1)));
    c.groupStart = reinterpret_cast<std::uint32_t*>(take(4 * (E + 1)));
    c.groupInfo = reinterpret_cast<std::uint32_t*>(take(4 * E));
    c.rowStartGroup = reinterpret_cast<std::uint32_t*>(take(4 * (E + 1)));
    c.wdCount = reinterpret_cast<std::uint32_t*>(take(4 * CW * 8));
    c.wdBase = reinterpret_cast<std::uint32_t*>(take(4 * CW * 8));
    c.wActive = reinterpret_cast<std::uint32_t*>(take(4 * CW));
    c.wTiles = reinterpret_cast<std::uint32_t*>(take(4 * CW));
    c.numRows = reinterpret_cast<std::uint32_t*>(take(4 * 4));
    const std::uint64_t tempElems =
        std::max({radix_temp_elems(E), scan_temp_elems(E + 1), scan_temp_elems(CW + 1), scan_temp_elems(SW + 1)});
    c.temp = reinterpret_cast<std::uint32_t*>(take(4 * tempElems));
    c.bytes = off;
    return c;
}

// ---------------------------------------------------------------- kernels

// buildEdgeKeysKernel (:104-144), with the super-window split folded into the
// key and range checks the reference does not make.
__global__ void build_keys_kernel(const std::uint32_t* __restrict__ dst, const std::uint32_t* __restrict__ src,
                                  std::uint32_t E, std::uint32_t rows, std::uint32_t cols, std::uint32_t S,
                                  unsigned wiBits, unsigned dstBits, std::uint64_t* __restrict__ keys,
                                  std::uint32_t* __restrict__ err) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    std::uint32_t s = src[e], d = dst[e];
    bool bad = false;
    if (s >= cols) {
        atomicMax(err, static_cast<std::uint32_t>(TCC_DEVERR_SRC_RANGE));
        bad = true;
    }
    if (rows != 0 && d >= rows) {
        atomicMax(err, static_cast<std::uint32_t>(TCC_DEVERR_DST_RANGE));
        bad = true;
    }
    if (bad) {  // keep every later index in range; the result is flagged invalid
        s = 0;
        d = 0;
    }
    const std::uint32_t w = s >> 3;
    const std::uint32_t sw = w / S;
    const std::uint32_t wi = w - sw * S;
    keys[e] = (((((static_cast<std::uint64_t>(sw) << dstBits) | d) << wiBits) | wi) << 3) | (s & 7u);
}

__global__ void group_flags_kernel(const std::uint64_t* __restrict__ keys, std::uint32_t E,
                                   std::uint32_t* __restrict__ flags) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    flags[e] = (e == 0 || (keys[e] >> 3) != (keys[e - 1] >> 3)) ? 1u : 0u;
}

// RLE of (window, dst) runs (the reference's DeviceRunLengthEncode, :1977-1990).
__global__ void group_emit_kernel(const std::uint64_t* __restrict__ keys, std::uint32_t E,
                                  const std::uint32_t* __restrict__ flags, const std::uint32_t* __restrict__ pos,
                                  std::uint64_t* __restrict__ groupKey, std::uint32_t* __restrict__ groupStart) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    if (flags[e]) {
        groupKey[pos[e]] = keys[e] >> 3;
        groupStart[pos[e]] = e;
    }
    if (e == E - 1) groupStart[pos[e] + flags[e]] = E;
}

// countWindowDegreesKernel (:147-213) + buildTileBitmapsKernel's row bits
// (:408-428) + the row-head flags of the distinct (super-window, dst) rows.
// A workgroup takes kFinalizeItems consecutive groups; groups are sorted by
// super-window, so they fall in at most a few super-windows, and the
// (window, degree) counts of its first two go to an LDS histogram flushed
// with one global atomic per nonzero bin (per-wave global atomics on the
// same 128 counters of a super-window serialised: 3.2 ms at 114M edges).
constexpr unsigned kFinalizeItems = 2048;
constexpr unsigned kFinalizeBins = TCC_SWTCF_MAX_SUPER_WINDOW_SIZE * 8;  // (wi, degree) of one super-window

__global__ void __launch_bounds__(kThreads) group_finalize_kernel(
    const std::uint64_t* __restrict__ keys, const std::uint64_t* __restrict__ groupKey,
    const std::uint32_t* __restrict__ groupStart, const std::uint32_t* __restrict__ numGroups, std::uint32_t E,
    std::uint32_t S, unsigned wiBits, unsigned dstBits, std::uint32_t* __restrict__ groupInfo,
    std::uint32_t* __restrict__ wdCount, std::uint32_t* __restrict__ rowFlags, std::uint32_t* __restrict__ err) {
    __shared__ std::uint32_t hist[2 * kFinalizeBins];
    for (unsigned i = threadIdx.x; i < 2 * kFinalizeBins; i += kThreads) hist[i] = 0;
    const std::uint32_t G = *numGroups;
    const std::uint32_t g0 = blockIdx.x * kFinalizeItems;
    const unsigned swShift = wiBits + dstBits;
    const std::uint32_t swFirst = g0 < G ? static_cast<std::uint32_t>(groupKey[g0] >> swShift) : 0u;
    __syncthreads();
    for (unsigned it = 0; it < kFinalizeItems / kThreads; ++it) {
        const std::uint32_t g = g0 + it * kThreads + threadIdx.x;
        if (g >= E) break;
        if (g >= G) {
            rowFlags[g] = 0;
            continue;
        }
        const std::uint32_t start = groupStart[g];
        const std::uint32_t count = groupStart[g + 1] - start;
        if (count == 0 || count > 8) atomicMax(err, static_cast<std::uint32_t>(TCC_DEVERR_DEGREE));
        const std::uint32_t deg = count == 0 ? 1u : (count > 8 ? 8u : count);
        std::uint32_t bits = 0;
        for (std::uint32_t i = 0; i < deg; ++i) bits |= 1u << static_cast<unsigned>(keys[start + i] & 7u);
        const std::uint64_t gk = groupKey[g];
        const std::uint32_t wi = static_cast<std::uint32_t>(gk & ((1ull << wiBits) - 1ull));
        const std::uint32_t sw = static_cast<std::uint32_t>(gk >> swShift);
        const std::uint32_t local = sw - swFirst;
        if (local < 2) {
            atomicAdd(&hist[local * kFinalizeBins + wi * 8 + deg - 1], 1u);
        } else {
            atomicAdd(&wdCount[(static_cast<std::uint64_t>(sw) * S + wi) * 8 + deg - 1], 1u);
        }
        groupInfo[g] = bits | (deg << 8);
        rowFlags[g] = (g == 0 || (gk >> wiBits) != (groupKey[g - 1] >> wiBits)) ? 1u : 0u;
    }
    __syncthreads();
    for (unsigned b = threadIdx.x; b < 2 * kFinalizeBins; b += kThreads) {
        const std::uint32_t n = hist[b];
        if (n == 0) continue;  // only bins of groups that exist (wi < S)
        const std::uint32_t sw = swFirst + b / kFinalizeBins;
        atomicAdd(&wdCount[static_cast<std::uint64_t>(sw) * S * 8 + (b % kFinalizeBins)], n);
    }
}

// buildWindowMetadataKernel (:216-265): degree 8 first, then 7 ... 1.
__global__ void window_meta_kernel(const std::uint32_t* __restrict__ wdCount, std::uint32_t* __restrict__ wdBase,
                                   std::uint32_t* __restrict__ wActive, std::uint32_t* __restrict__ wTiles,
                                   std::uint32_t CW) {
    const std::uint32_t w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= CW) return;
    std::uint32_t running = 0;
    for (int d = 7; d >= 0; --d) {
        const std::uint64_t i = static_cast<std::uint64_t>(w) * 8 + d;
        wdBase[i] = running;
        running += wdCount[i];
    }
    wActive[w] = running;
    wTiles[w] = (running + 7) / 8;
}

// Distinct (super-window, dst) rows: superWindowRows in slot order and the
// per-super-window row counts (the reference's hash insert + slot assignment,
// :459-681, as a sorted run encoding).
__global__ void row_emit_kernel(const std::uint64_t* __restrict__ groupKey,
                                const std::uint32_t* __restrict__ rowFlags, const std::uint32_t* __restrict__ rowPos,
                                const std::uint32_t* __restrict__ numGroups, std::uint32_t E, unsigned wiBits,
                                unsigned dstBits, std::uint32_t numSuperWindows,
                                std::uint32_t* __restrict__ rowStartGroup,
                                std::uint32_t* __restrict__ superWindowRows,
                                std::uint32_t* __restrict__ superWindowRowOffset) {
    const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= E) return;
    const std::uint32_t G = *numGroups;
    if (g >= G) return;
    const unsigned swShift = wiBits + dstBits;
    if (rowFlags[g]) {
        const std::uint32_t u = rowPos[g];
        const std::uint64_t gk = groupKey[g];
        const std::uint32_t dstMask = dstBits >= 32 ? 0xFFFFFFFFu : ((1u << dstBits) - 1u);
        const std::uint32_t d = static_cast<std::uint32_t>(gk >> wiBits) & dstMask;
        const std::uint32_t sw = static_cast<std::uint32_t>(gk >> swShift);
        rowStartGroup[u] = g;
        superWindowRows[u] = d;
        // Rows are sorted by super-window: the first row of super-window sw
        // sets its offset, and those of the empty super-windows before it.
        const std::int64_t prev = g == 0 ? -1 : static_cast<std::int64_t>(groupKey[g - 1] >> swShift);
        for (std::int64_t t = prev + 1; t <= static_cast<std::int64_t>(sw) && t < numSuperWindows; ++t)
            superWindowRowOffset[t] = u;
    }
    if (g == G - 1) {
        const std::uint32_t U = rowPos[g] + rowFlags[g];
        rowStartGroup[U] = G;
        const std::uint32_t sw = static_cast<std::uint32_t>(groupKey[g] >> swShift);
        for (std::uint32_t t = sw + 1; t <= numSuperWindows; ++t) superWindowRowOffset[t] = U;
    }
}

// Stable rank of `bin` among the active items of a 256-item chunk (item order
// = thread order), continuing the running per-bin counts in `run`.  Must be
// called by all threads of the block.  `wcnt` is zero on entry and on exit.
template <int NBITS, unsigned THREADS>
__device__ std::uint32_t block_multisplit_rank(unsigned bin, bool active, std::uint32_t* run,
                                               std::uint32_t (*wcnt)[256]) {
    const unsigned wave = threadIdx.x / kWave;
    const std::uint64_t lt = lanemask_lt();
    const std::uint64_t peers = match_peers<NBITS>(bin, active);
    const std::uint32_t rin = static_cast<std::uint32_t>(__popcll(peers & lt));
    if (active && (peers & lt) == 0) wcnt[wave][bin] = static_cast<std::uint32_t>(__popcll(peers));
    __syncthreads();
    std::uint32_t rank = 0;
    if (active) {
        std::uint32_t cross = 0;
        for (unsigned w = 0; w < wave; ++w) cross += wcnt[w][bin];
        rank = run[bin] + cross + rin;
    }
    __syncthreads();
    for (unsigned b = threadIdx.x; b < (1u << NBITS); b += blockDim.x) {
        std::uint32_t t = 0;
        for (int w = 0; w < static_cast<int>(THREADS / kWave); ++w) {
            t += wcnt[w][b];
            wcnt[w][b] = 0;
        }
        run[b] += t;
    }
    __syncthreads();
    return rank;
}

// One workgroup per super-window:
//  (a) assignGroupLocationsKernel (:292-376) with the canonical rank,
//      fillValidTileRowSlotsKernel (:1003-1048) and the tile bitmaps
//      (:430-455, written as one byte per tile row instead of atomicOr);
//  (b) buildRepeatCacheMetadataKernel (:699-895) with the canonical order.
template <unsigned THREADS>
__global__ void __launch_bounds__(THREADS) super_window_kernel(
    const std::uint64_t* __restrict__ groupKey, const std::uint32_t* __restrict__ groupInfo,
    const std::uint32_t* __restrict__ rowFlags, const std::uint32_t* __restrict__ rowPos,
    const std::uint32_t* __restrict__ rowStartGroup, const std::uint32_t* __restrict__ wdBase,
    const std::uint32_t* __restrict__ colWindowOffset, const std::uint32_t* __restrict__ superWindowRowOffset,
    std::uint32_t S, unsigned wiBits, std::uint32_t numColWindows, std::uint32_t* __restrict__ tileRowSlot,
    std::uint8_t* __restrict__ tileBytes, std::uint8_t* __restrict__ rowCacheSlot,
    std::uint32_t* __restrict__ cachedRowSlot, std::uint8_t* __restrict__ cachedCount,
    std::uint32_t* __restrict__ err) {
    __shared__ std::uint32_t run[256];
    __shared__ std::uint32_t wcnt[THREADS / kWave][256];
    __shared__ std::uint32_t occHist[TCC_SWTCF_MAX_SUPER_WINDOW_SIZE + 1];
    __shared__ std::uint32_t occBase[TCC_SWTCF_MAX_SUPER_WINDOW_SIZE + 1];
    __shared__ std::uint32_t repeatedTotal;

    const std::uint32_t s = blockIdx.x;
    const std::uint32_t off0 = superWindowRowOffset[s];
    const std::uint32_t off1 = superWindowRowOffset[s + 1];
    const std::uint32_t g0 = rowStartGroup[off0];
    const std::uint32_t g1 = rowStartGroup[off1];
    const std::uint64_t wiMask = (1ull << wiBits) - 1ull;

    for (unsigned i = threadIdx.x; i < 256; i += THREADS) {
        run[i] = 0;
        for (int w = 0; w < static_cast<int>(THREADS / kWave); ++w) wcnt[w][i] = 0;
    }
    if (threadIdx.x <= TCC_SWTCF_MAX_SUPER_WINDOW_SIZE) occHist[threadIdx.x] = 0;
    __syncthreads();

    // (a) rows of every window of this super-window
    for (std::uint32_t base = g0; base < g1; base += THREADS) {
        const std::uint32_t g = base + threadIdx.x;
        const bool active = g < g1;
        std::uint32_t info = 0, wi = 0, deg = 1;
        if (active) {
            info = groupInfo[g];
            wi = static_cast<std::uint32_t>(groupKey[g] & wiMask);
            deg = info >> 8;
        }
        const unsigned bin = wi * 8 + (deg - 1);
        const std::uint32_t rank = block_multisplit_rank<8, THREADS>(bin, active, run, wcnt);
        if (active) {
            const std::uint32_t w = s * S + wi;
            if (w < numColWindows) {
                const std::uint32_t reordered = wdBase[static_cast<std::uint64_t>(w) * 8 + deg - 1] + rank;
                const std::uint64_t loc = static_cast<std::uint64_t>(colWindowOffset[w] + reordered / 8) * 8 +
                                          (reordered & 7u);
                const std::uint32_t u = rowPos[g] + rowFlags[g] - 1;
                tileRowSlot[loc] = u - off0;
                tileBytes[loc] = static_cast<std::uint8_t>(info & 0xFFu);
            }
        }
    }

    // (b) repeat cache: occurrence histogram, descending bases, stable ranks
    for (std::uint32_t u = off0 + threadIdx.x; u < off1; u += THREADS) {
        const std::uint32_t occ = rowStartGroup[u + 1] - rowStartGroup[u];
        if (occ > TCC_SWTCF_MAX_SUPER_WINDOW_SIZE) {
            atomicMax(err, static_cast<std::uint32_t>(TCC_DEVERR_OCCURRENCE));
        } else if (occ > 1) {
            atomicAdd(&occHist[occ], 1u);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        std::uint32_t running = 0;
        for (int o = TCC_SWTCF_MAX_SUPER_WINDOW_SIZE; o >= 2; --o) {
            occBase[o] = running;
            running += occHist[o];
        }
        repeatedTotal = running;
        cachedCount[s] = static_cast<std::uint8_t>(running < TCC_SWTCF_REPEAT_CACHE_SIZE
                                                       ? running
                                                       : TCC_SWTCF_REPEAT_CACHE_SIZE);
    }
    for (unsigned i = threadIdx.x; i < 256; i += THREADS) run[i] = 0;
    __syncthreads();
    if (repeatedTotal == 0) return;  // uniform across the block
    for (std::uint32_t base = off0; base < off1; base += THREADS) {
        const std::uint32_t u = base + threadIdx.x;
        std::uint32_t occ = 0;
        if (u < off1) occ = rowStartGroup[u + 1] - rowStartGroup[u];
        const bool rep = u < off1 && occ > 1 && occ <= TCC_SWTCF_MAX_SUPER_WINDOW_SIZE;
        const std::uint32_t rank = block_multisplit_rank<6, THREADS>(rep ? occ : 0u, rep, run, wcnt);
        if (rep) {
            const std::uint32_t cs = occBase[occ] + rank;
            if (cs < TCC_SWTCF_REPEAT_CACHE_SIZE) {
                rowCacheSlot[u] = static_cast<std::uint8_t>(cs);
                cachedRowSlot[static_cast<std::uint64_t>(s) * TCC_SWTCF_REPEAT_CACHE_SIZE + cs] = u - off0;
            }
        }
    }
}

// fillPaddingTileRowSlotsKernel (:1051-1107).
__global__ void padding_kernel(const std::uint32_t* __restrict__ wActive,
                               const std::uint32_t* __restrict__ colWindowOffset, std::uint32_t CW,
                               std::uint32_t* __restrict__ tileRowSlot) {
    const std::uint32_t w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= CW) return;
    const std::uint32_t active = wActive[w];
    const std::uint32_t rem = active & 7u;
    if (active == 0 || rem == 0) return;
    const std::uint64_t last = colWindowOffset[w + 1] - 1;
    for (std::uint32_t lr = rem; lr < 8; ++lr) tileRowSlot[last * 8 + lr] = TCC_SWTCF_INVALID_ROW_SLOT;
}

}  // namespace
}  // namespace tcc

using namespace tcc;

extern "C" {

int tcc_swtcf_alloc_matrix(tcc_swtcf_matrix* m, std::uint32_t rows, std::uint32_t cols, std::uint32_t nnz,
                           std::uint32_t superWindowSize) {
    clear_last_error();
    TCC_REQUIRE(m != nullptr, TCC_ERR_INVALID_ARGUMENT, "matrix is null");
    TCC_REQUIRE(cols != 0 && nnz != 0 && superWindowSize != 0 &&
                    superWindowSize <= TCC_SWTCF_MAX_SUPER_WINDOW_SIZE,
                TCC_ERR_INVALID_ARGUMENT, "invalid SWTCF allocation size");
    std::memset(m, 0, sizeof(*m));
    m->rows = rows;
    m->cols = cols;
    m->nnz = nnz;
    m->colWindowWidth = TCC_SWTCF_COL_WINDOW_WIDTH;
    m->tileRows = TCC_SWTCF_TILE_ROWS;
    m->superWindowSize = superWindowSize;
    m->numColWindows = (cols + TCC_SWTCF_COL_WINDOW_WIDTH - 1) / TCC_SWTCF_COL_WINDOW_WIDTH;
    m->numSuperWindows = (m->numColWindows + superWindowSize - 1) / superWindowSize;
    const std::size_t E = nnz, SW = m->numSuperWindows, CW = m->numColWindows;
    // One allocation carved in the reference's array order (:1166-1262).
    const std::size_t sizes[8] = {4 * (SW + 1), 4 * E, E, 4 * SW * 32, SW, 4 * (CW + 1), 4 * E * 8, 8 * E};
    std::size_t total = 0;
    for (std::size_t s : sizes) total += align_up(s);
    char* base = nullptr;
    if (hipMalloc(&base, total) != hipSuccess) {
        std::memset(m, 0, sizeof(*m));
        set_last_error("hipMalloc failed for the SWTCF arrays");
        return TCC_ERR_NO_MEMORY;
    }
    std::size_t off = 0;
    char* p[8];
    for (int i = 0; i < 8; ++i) {
        p[i] = base + off;
        off += align_up(sizes[i]);
    }
    m->superWindowRowOffset = reinterpret_cast<std::uint32_t*>(p[0]);
    m->superWindowRows = reinterpret_cast<std::uint32_t*>(p[1]);
    m->superWindowRowCacheSlot = reinterpret_cast<std::uint8_t*>(p[2]);
    m->superWindowCachedRowSlot = reinterpret_cast<std::uint32_t*>(p[3]);
    m->superWindowCachedCount = reinterpret_cast<std::uint8_t*>(p[4]);
    m->colWindowOffset = reinterpret_cast<std::uint32_t*>(p[5]);
    m->tileRowSlot = reinterpret_cast<std::uint32_t*>(p[6]);
    m->tileLocalBit = reinterpret_cast<std::uint64_t*>(p[7]);
    return TCC_OK;
}

int tcc_swtcf_free_matrix(tcc_swtcf_matrix* m) {
    clear_last_error();
    if (!m) return TCC_OK;
    if (m->superWindowRowOffset) TCC_HIP_CHECK(hipFree(m->superWindowRowOffset));
    std::memset(m, 0, sizeof(*m));
    return TCC_OK;
}

int tcc_swtcf_alloc_workspace(tcc_swtcf_workspace* ws, std::uint32_t edgeCapacity, std::uint32_t numSrc,
                              std::uint32_t superWindowSize) {
    clear_last_error();
    TCC_REQUIRE(ws != nullptr, TCC_ERR_INVALID_ARGUMENT, "workspace is null");
    TCC_REQUIRE(edgeCapacity != 0 && numSrc != 0 && superWindowSize != 0 &&
                    superWindowSize <= TCC_SWTCF_MAX_SUPER_WINDOW_SIZE,
                TCC_ERR_INVALID_ARGUMENT, "invalid converter workspace size");
    std::memset(ws, 0, sizeof(*ws));
    ws->edgeCapacity = edgeCapacity;
    ws->numColWindows = (numSrc + 7) / 8;
    ws->numSuperWindows = (ws->numColWindows + superWindowSize - 1) / superWindowSize;
    ws->superWindowSize = superWindowSize;
    const Carve c = carve(nullptr, edgeCapacity, ws->numColWindows, ws->numSuperWindows);
    const std::size_t bytes = c.bytes + 256;  // + deviceNumGroups / deviceError
    char* base = nullptr;
    if (hipMalloc(&base, bytes) != hipSuccess) {
        std::memset(ws, 0, sizeof(*ws));
        set_last_error("hipMalloc failed for the converter workspace");
        return TCC_ERR_NO_MEMORY;
    }
    ws->scratch = base;
    ws->scratchBytes = bytes;
    ws->deviceNumGroups = reinterpret_cast<std::uint32_t*>(base + c.bytes);
    ws->deviceError = ws->deviceNumGroups + 1;
    TCC_HIP_CHECK(hipMemset(ws->deviceNumGroups, 0, 8));
    return TCC_OK;
}

int tcc_swtcf_free_workspace(tcc_swtcf_workspace* ws) {
    clear_last_error();
    if (!ws) return TCC_OK;
    if (ws->scratch) TCC_HIP_CHECK(hipFree(ws->scratch));
    std::memset(ws, 0, sizeof(*ws));
    return TCC_OK;
}

int tcc_swtcf_convert(const std::uint32_t* dDst, const std::uint32_t* dSrc, std::uint32_t numEdges,
                      tcc_swtcf_matrix* m, tcc_swtcf_workspace* ws, void* streamArg) {
    clear_last_error();
    TCC_REQUIRE(m && ws && dDst && dSrc, TCC_ERR_INVALID_ARGUMENT, "null argument");
    TCC_REQUIRE(numEdges != 0 && numEdges <= ws->edgeCapacity && numEdges <= m->nnz &&
                    m->colWindowWidth == TCC_SWTCF_COL_WINDOW_WIDTH && m->tileRows == TCC_SWTCF_TILE_ROWS &&
                    m->superWindowSize != 0 && m->superWindowSize <= TCC_SWTCF_MAX_SUPER_WINDOW_SIZE,
                TCC_ERR_INVALID_ARGUMENT, "invalid COO -> SWTCF conversion arguments");
    TCC_REQUIRE(ws->numColWindows >= m->numColWindows && ws->superWindowSize == m->superWindowSize,
                TCC_ERR_INVALID_ARGUMENT, "workspace was sized for a different matrix");
    const hipStream_t st = as_stream(streamArg);
    const std::uint32_t E = numEdges, CW = m->numColWindows, SW = m->numSuperWindows, S = m->superWindowSize;
    const KeyLayout kl = key_layout(m->rows, S, SW);
    TCC_REQUIRE(kl.total <= 64, TCC_ERR_UNSUPPORTED, "packed sort key exceeds 64 bits");
    const Carve c = carve(static_cast<char*>(ws->scratch), ws->edgeCapacity, ws->numColWindows,
                          ws->numSuperWindows);
    std::uint32_t* err = ws->deviceError;
    std::uint32_t* numGroups = ws->deviceNumGroups;

    // Reset per-conversion state (:1789-1919), with fill kernels.
    TCC_HIP_CHECK(fill<std::uint64_t>(m->tileLocalBit, m->nnz, 0ull, st));
    TCC_HIP_CHECK(fill<std::uint8_t>(m->superWindowRowCacheSlot, m->nnz, 0xFFu, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(m->superWindowCachedRowSlot, static_cast<std::uint64_t>(SW) * 32,
                                      0xFFFFFFFFu, st));
    TCC_HIP_CHECK(fill<std::uint8_t>(m->superWindowCachedCount, SW, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(c.wdCount, static_cast<std::uint64_t>(CW) * 8, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(m->superWindowRowOffset, static_cast<std::uint64_t>(SW) + 1, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(err, 1, 0u, st));

    // 1-2. keys, sort
    hipLaunchKernelGGL(build_keys_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, dDst, dSrc, E,
                       m->rows, m->cols, S, kl.wiBits, kl.dstBits, c.keysA, err);
    TCC_LAUNCH_CHECK();
    std::uint64_t* sorted = nullptr;
    TCC_HIP_CHECK(radix_sort(c.keysA, c.keysB, E, kl.total, c.temp, &sorted, st));
    std::uint64_t* groupKey = (sorted == c.keysA) ? c.keysB : c.keysA;

    // 3. groups
    hipLaunchKernelGGL(group_flags_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, E,
                       c.flags);
    TCC_LAUNCH_CHECK();
    TCC_HIP_CHECK(exclusive_scan(c.flags, c.pos, E, numGroups, c.temp, st));
    hipLaunchKernelGGL(group_emit_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, E,
                       c.flags, c.pos, groupKey, c.groupStart);
    TCC_LAUNCH_CHECK();
    hipLaunchKernelGGL(group_finalize_kernel, dim3(grid_for(E, kFinalizeItems)), dim3(kThreads), 0, st, sorted,
                       groupKey, c.groupStart, numGroups, E, S, kl.wiBits, kl.dstBits, c.groupInfo, c.wdCount,
                       c.flags, err);
    TCC_LAUNCH_CHECK();

    // 4-5. window metadata, colWindowOffset
    hipLaunchKernelGGL(window_meta_kernel, dim3(grid_for(CW, kThreads)), dim3(kThreads), 0, st, c.wdCount,
                       c.wdBase, c.wActive, c.wTiles, CW);
    TCC_LAUNCH_CHECK();
    TCC_HIP_CHECK(exclusive_scan(c.wTiles, m->colWindowOffset, CW, m->colWindowOffset + CW, c.temp, st));

    // 8-10. distinct super-window rows, superWindowRowOffset
    TCC_HIP_CHECK(exclusive_scan(c.flags, c.pos, E, c.numRows, c.temp, st));
    hipLaunchKernelGGL(row_emit_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, groupKey, c.flags,
                       c.pos, numGroups, E, kl.wiBits, kl.dstBits, SW, c.rowStartGroup, m->superWindowRows,
                       m->superWindowRowOffset);
    TCC_LAUNCH_CHECK();

    // 6-7, 11-13. per super-window: row locations, slots, bitmaps, cache
    // Super-windows with many groups (63k on average at 114M edges) walk them
    // 1024 at a time; small ones keep 256-thread workgroups.
    auto sw_launch = [&](auto kernel, unsigned threads) {
        hipLaunchKernelGGL(kernel, dim3(SW), dim3(threads), 0, st, groupKey, c.groupInfo, c.flags, c.pos,
                           c.rowStartGroup, c.wdBase, m->colWindowOffset, m->superWindowRowOffset, S, kl.wiBits, CW,
                           m->tileRowSlot, reinterpret_cast<std::uint8_t*>(m->tileLocalBit),
                           m->superWindowRowCacheSlot, m->superWindowCachedRowSlot, m->superWindowCachedCount, err);
    };
    if (E / std::max<std::uint64_t>(SW, 1) >= 8192) sw_launch(super_window_kernel<1024>, 1024);
    else sw_launch(super_window_kernel<kThreads>, kThreads);
    TCC_LAUNCH_CHECK();
    hipLaunchKernelGGL(padding_kernel, dim3(grid_for(CW, kThreads)), dim3(kThreads), 0, st, c.wActive,
                       m->colWindowOffset, CW, m->tileRowSlot);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

}  // extern "C"
