// Dense hub tiles on MFMA plus a sparse remainder, for gfx950 (no reference
// counterpart; the product is the one tf32_spmm_bcsr computes,
// spmm_cnic/src/core/spmm_kernel.cu:1560-1842, with its mma.m16n8k8 TF32
// numerics).
//
// Skewed (R-MAT) graphs hide a dense core: with rows and columns each
// ordered by degree (descending, ties by index), the 16x16 tiles of the
// reordered matrix near its top-left corner are mostly full.  At the
// 233k-node, 114M-nnz configuration, 567k tiles hold at least 32 nonzeros
// (54M nonzeros, 47%), against about one nonzero per column in the 8x8
// blocks of the BCSR.  Those tiles are stored densely (TF32-rounded values,
// zeros included) in the order of the MFMA A operand and multiplied with
// v_mfma_f32_16x16x4f32; every other entry goes to an ordinary (phased)
// BCSR and the gather kernels.
//
// Tile format: row block b = degree-sorted rows 16b..16b+15 (rowOrder gives
// their original indices); its tiles are [rowBlockOffset[b],
// rowBlockOffset[b+1]), tile t covering column ranks 16*tileCol[t] .. +15.
// tileVals[256t + 4l + s] = A(row l%16, column 4s + l/16) of tile t: lane l's
// A operand of MFMA step s (lane l supplies A(i = l%16, k = l/16), B(k = l/16,
// j = l%16) and holds D(4*(l/16) + v, l%16) in register v).
//
// SpMM: the feature rows of the hub columns (ranks < hub_cols) are copied in
// rank order, TF32-rounded, into a workspace of rows padded to 64 features
// (Xh).  One wave per (unit of at most unit_tiles tiles of one row block,
// 64-feature slice): per tile one float4 of A and four float4 of Xh (four
// rows of 64 features), and 16 MFMAs into 4 accumulator tiles (the N tile u
// of lane l is feature 4*(l%16) + u, so one float4 of Xh feeds all four).
// The remainder's gather runs first and fills Y; the tiles are added into
// it (stores for a row block held by one unit, fp32 atomics otherwise).
#include <algorithm>
#include <cstring>

#include "../../include/tcc_spmm_cnic.h"
#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "degree_rank.hpp"
#include "primitives.hpp"

namespace tcc {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr std::uint32_t kTile = 16;
constexpr std::uint32_t kTileVals = kTile * kTile;  // floats per tile
constexpr std::uint32_t kSlice = 64;                // features per wave
constexpr std::uint32_t kDefaultUnitTiles = 32;
constexpr std::uint32_t kMaxUnitTiles = 64;         // a unit's tile columns sit one per lane
constexpr int kStages = 3;                          // tiles in flight per wave, the current one included
constexpr std::uint32_t kDefaultMinTileNnz = 32;
constexpr unsigned kThreads = 256;

inline std::size_t align_up(std::size_t x) { return (x + 255) & ~std::size_t(255); }

// ---------------------------------------------------------------- builder

// key = (row block * column blocks + column block) << 8 | (row % 16) << 4 |
// (column rank % 16); payload = edge.
__global__ void tile_keys_kernel(const std::uint32_t* __restrict__ row, const std::uint32_t* __restrict__ col,
                                 std::uint32_t E, const std::uint32_t* __restrict__ rowRank,
                                 const std::uint32_t* __restrict__ colRank, std::uint32_t colBlocks,
                                 std::uint64_t* __restrict__ keys, std::uint32_t* __restrict__ perm) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint32_t rr = rowRank[row[e]], cr = colRank[col[e]];
    const std::uint64_t tile = static_cast<std::uint64_t>(rr / kTile) * colBlocks + cr / kTile;
    keys[e] = tile << 8 | (rr % kTile) << 4 | (cr % kTile);
    perm[e] = e;
}

// Tile heads; a repeated full key is a duplicate edge.
__global__ void tile_heads_kernel(const std::uint64_t* __restrict__ keys, std::uint32_t E,
                                  std::uint32_t* __restrict__ flags, std::uint32_t* __restrict__ err) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint64_t k = keys[e];
    flags[e] = (e == 0 || (k >> 8) != (keys[e - 1] >> 8)) ? 1u : 0u;
    if (e > 0 && k == keys[e - 1]) atomicMax(err, 2u);
}

__global__ void tile_start_kernel(const std::uint32_t* __restrict__ flags, const std::uint32_t* __restrict__ pos,
                                  std::uint32_t E, std::uint32_t* __restrict__ tileStart) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < E && flags[e]) tileStart[pos[e]] = e;
}

// dense[t] = tile t holds at least minNnz entries; per row block, its dense
// tiles; the largest column block of a dense tile (+1).
__global__ void dense_tiles_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ tileStart,
                                   const std::uint32_t* __restrict__ numTiles, std::uint32_t E, std::uint32_t minNnz,
                                   std::uint32_t colBlocks, std::uint32_t* __restrict__ dense,
                                   std::uint32_t* __restrict__ blockTiles, std::uint32_t* __restrict__ hubBlocks) {
    const std::uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= *numTiles) return;
    const std::uint32_t s = tileStart[t];
    const std::uint32_t e = t + 1 < *numTiles ? tileStart[t + 1] : E;
    const bool d = e - s >= minNnz;
    dense[t] = d ? 1u : 0u;
    if (d) {
        const std::uint64_t tile = keys[s] >> 8;
        atomicAdd(&blockTiles[tile / colBlocks], 1u);
        atomicMax(hubBlocks, static_cast<std::uint32_t>(tile % colBlocks) + 1u);
    }
}

// Per edge: 1 if it stays in the sparse remainder.
__global__ void rest_flags_kernel(const std::uint32_t* __restrict__ flags, const std::uint32_t* __restrict__ pos,
                                  const std::uint32_t* __restrict__ dense, std::uint32_t E,
                                  std::uint32_t* __restrict__ rest) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < E) rest[e] = dense[pos[e] + flags[e] - 1] ? 0u : 1u;
}

__global__ void units_per_block_kernel(const std::uint32_t* __restrict__ blockTiles, std::uint32_t RB,
                                       std::uint32_t unitTiles, std::uint32_t* __restrict__ units) {
    const std::uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < RB) units[b] = (blockTiles[b] + unitTiles - 1) / unitTiles;
}

// Dense tiles' values (TF32-rounded) into the A-operand order, the others
// into the remainder COO.
__global__ void place_entries_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ perm,
                                     std::uint32_t E, const std::uint32_t* __restrict__ flags,
                                     const std::uint32_t* __restrict__ pos, const std::uint32_t* __restrict__ dense,
                                     const std::uint32_t* __restrict__ denseId,
                                     const std::uint32_t* __restrict__ restPos, const std::uint32_t* __restrict__ row,
                                     const std::uint32_t* __restrict__ col, const float* __restrict__ val,
                                     float* __restrict__ tileVals, std::uint32_t* __restrict__ restRow,
                                     std::uint32_t* __restrict__ restCol, float* __restrict__ restVal) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint32_t t = pos[e] + flags[e] - 1;
    const std::uint32_t src = perm[e];
    const float v = val ? val[src] : 1.0f;
    if (dense[t]) {
        const std::uint32_t i = static_cast<std::uint32_t>(keys[e] >> 4) & 15u, j = static_cast<std::uint32_t>(keys[e]) & 15u;
        const std::uint32_t lane = i + 16 * (j % 4), step = j / 4;
        tileVals[static_cast<std::uint64_t>(denseId[t]) * kTileVals + 4 * lane + step] = tf32_rna(v);
    } else {
        const std::uint32_t p = restPos[e];
        restRow[p] = row[src];
        restCol[p] = col[src];
        if (restVal) restVal[p] = v;
    }
}

__global__ void tile_cols_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ tileStart,
                                 const std::uint32_t* __restrict__ numTiles, const std::uint32_t* __restrict__ dense,
                                 const std::uint32_t* __restrict__ denseId, std::uint32_t colBlocks,
                                 std::uint32_t* __restrict__ tileCol) {
    const std::uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < *numTiles && dense[t]) tileCol[denseId[t]] = static_cast<std::uint32_t>((keys[tileStart[t]] >> 8) % colBlocks);
}

// units[3u .. 3u+2] = row block, first tile, end tile.
__global__ void tile_units_kernel(const std::uint32_t* __restrict__ rowBlockOffset,
                                  const std::uint32_t* __restrict__ unitFirst, std::uint32_t RB, std::uint32_t unitTiles,
                                  std::uint32_t* __restrict__ units) {
    const std::uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= RB) return;
    const std::uint32_t t0 = rowBlockOffset[b], t1 = rowBlockOffset[b + 1];
    for (std::uint32_t k = 0; unitFirst[b] + k < unitFirst[b + 1]; ++k) {
        const std::uint64_t u = 3ull * (unitFirst[b] + k);
        units[u] = b;
        units[u + 1] = t0 + k * unitTiles;
        units[u + 2] = min(t0 + (k + 1) * unitTiles, t1);
    }
}

template <typename T>
struct DevBuf {
    T* p = nullptr;
    ~DevBuf() {
        if (p) (void)hipFree(p);
    }
};

// ---------------------------------------------------------------- SpMM

// Xh[r][f] = TF32(X[hubColOrder[r]][f]) for f < F, 0 for F <= f < ldh.
__global__ void hub_rows_kernel(const float* __restrict__ X, std::uint32_t F, const std::uint32_t* __restrict__ order,
                                std::uint32_t hubCols, std::uint32_t ldh, float* __restrict__ Xh) {
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::uint32_t r = static_cast<std::uint32_t>(i / ldh), f = static_cast<std::uint32_t>(i % ldh);
    if (r >= hubCols) return;
    Xh[i] = f < F ? tf32_rna(X[static_cast<std::uint64_t>(order[r]) * F + f]) : 0.0f;
}

struct TileArgs {
    const std::uint32_t* rowOrder;
    const std::uint32_t* rowBlockOffset;
    const std::uint32_t* tileCol;
    const float* tileVals;
    const std::uint32_t* units;
    const float* Xh;
    std::uint32_t ldh;  // Xh row stride (a multiple of 64)
    float* Y;
    float* partials;    // [num_units][16][ldh]: sums of the units of shared row blocks
    std::uint32_t F;
    std::uint32_t numUnits;
    std::uint32_t slices;
    std::uint32_t unitTiles;
};

// One tile's operands for one wave: A (lane l: A(l%16, 4s + l/16), s = 0..3)
// and four 4-row steps of Xh (lane l: row 4s + l/16, features 4(l%16)..+3).
struct TileOperands {
    f32x4 a;
    f32x4 b[4];
};

// Row r (0..15) of row block b in Y, or nullptr for the padding of the
// last block.
__device__ __forceinline__ float* y_row(const TileArgs& a, std::uint32_t b, unsigned r) {
    const std::uint32_t orow = a.rowOrder[static_cast<std::uint64_t>(b) * kTile + r];
    return orow == TCC_SWTCF_INVALID_ROW_SLOT ? nullptr : a.Y + static_cast<std::uint64_t>(orow) * a.F;
}

// Y[row][f..f+3] += s (features below F only).
__device__ __forceinline__ void add_quad(float* row, std::uint32_t f, std::uint32_t F, bool vec, const f32x4& s) {
    if (!row || f >= F) return;
    float* out = row + f;
    if (vec) {
        f32x4 y = load_global<vf4>(out);
        y += s;
        *reinterpret_cast<f32x4*>(out) = y;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (f + u < F) out[u] += s[u];
    }
}

// One wave per (unit of at most 64 tiles of one row block, 64-feature
// slice), unit-major, so the waves of one unit (one workgroup for F <= 256)
// read the same tiles.  The unit's tile columns sit one per lane and are read
// with readlane; operands are loaded NS - 1 tiles ahead into a ring of NS
// stages, every load unconditional (clamped to the unit's last tile): loads
// complete in order, so a conditional load, a copy between stages or a
// branch out of the ring would make the wave wait for the newest one; the
// last trip's tiles past the unit's end multiply a zero A instead.  A row
// block held by one unit adds its sums into Y; the units of a shared row
// block store theirs in `partials` for hub_reduce_kernel (no atomics, and a
// sum order that does not depend on scheduling).
template <int NS>
__global__ void __launch_bounds__(kThreads) hub_tiles_kernel(TileArgs a) {
    const unsigned lane = __lane_id();
    const std::uint32_t w = blockIdx.x * (kThreads / kWave) +
                            static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave)));
    const std::uint32_t unit = w / a.slices, slice = w - unit * a.slices;
    if (unit >= a.numUnits) return;
    const std::uint32_t b = a.units[3ull * unit], t0 = a.units[3ull * unit + 1], t1 = a.units[3ull * unit + 2];
    if (t0 >= t1) return;
    const bool shared = t0 != a.rowBlockOffset[b] || t1 != a.rowBlockOffset[b + 1];
    const std::uint32_t f0 = slice * kSlice;
    const unsigned li = lane & 15u, lk = lane >> 4;
    const std::uint32_t last = t1 - 1;
    const int cols = static_cast<int>(a.tileCol[min(t0 + lane, last)]);
    // this lane's B element offset in a 4-row step: row lk, features 4*li..+3
    const float* xb = a.Xh + static_cast<std::uint64_t>(lk) * a.ldh + f0 + 4 * li;
    const float* av = a.tileVals + 4 * lane;

    auto load = [&](std::uint32_t t, TileOperands& o) {
        const std::uint32_t col = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(cols, static_cast<int>(t - t0)));
        o.a = load_global<vf4>(av + static_cast<std::uint64_t>(t) * kTileVals);
        const float* rb = xb + static_cast<std::uint64_t>(col) * kTile * a.ldh;
#pragma unroll
        for (int s = 0; s < 4; ++s) o.b[s] = load_global<vf4>(rb + static_cast<std::uint64_t>(4 * s) * a.ldh);
    };
    f32x4 acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    // a tile past the unit's end (the ring's tail) adds A = 0
    auto mma = [&](const TileOperands& o, bool live) {
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const float as = live ? o.a[s] : 0.0f;
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(as, o.b[s][u], acc[u], 0, 0, 0);
        }
    };

    TileOperands ring[NS];
#pragma unroll
    for (int j = 0; j < NS - 1; ++j) {
        load(min(t0 + j, last), ring[j]);
        __builtin_amdgcn_sched_barrier(0);  // stage j's loads before stage j+1's
    }
    for (std::uint32_t t = t0; t < t1; t += NS) {
#pragma unroll
        for (int j = 0; j < NS; ++j) {
            load(min(t + j + NS - 1, last), ring[(j + NS - 1) % NS]);
            // keep the loads ahead of the products (the scheduler would
            // sink them next to their use to save registers)
            __builtin_amdgcn_sched_barrier(0);
            mma(ring[j], t + j < t1);
        }
    }

    // D(4*lk + v, li) of N tile u: row 16b + 4*lk + v, feature f0 + 4*li + u.
    const std::uint32_t f = f0 + 4 * li;
    if (shared) {
        float* p = a.partials + (static_cast<std::uint64_t>(unit) * kTile + 4 * lk) * a.ldh + f;
#pragma unroll
        for (int v = 0; v < 4; ++v)
            *reinterpret_cast<f32x4*>(p + static_cast<std::uint64_t>(v) * a.ldh) =
                f32x4{acc[0][v], acc[1][v], acc[2][v], acc[3][v]};
        return;
    }
    const bool vec = a.F % 4 == 0 && (reinterpret_cast<std::uintptr_t>(a.Y) & 15u) == 0;
#pragma unroll
    for (int v = 0; v < 4; ++v)
        add_quad(y_row(a, b, 4 * lk + v), f, a.F, vec, f32x4{acc[0][v], acc[1][v], acc[2][v], acc[3][v]});
}

// Y rows of a shared row block += the sum of its units' partials, one
// workgroup per (unit, slice) of which only the row block's first unit
// works: thread q sums row q/16, features 4(q%16)..+3 of the slice over the
// block's units (ceil(tiles / unitTiles) of them, consecutive), eight loads
// in flight.
__global__ void __launch_bounds__(kThreads) hub_reduce_kernel(TileArgs a) {
    const std::uint32_t unit = blockIdx.x / a.slices, slice = blockIdx.x - unit * a.slices;
    const std::uint32_t b = a.units[3ull * unit], t0 = a.units[3ull * unit + 1];
    const std::uint32_t tb0 = a.rowBlockOffset[b], tb1 = a.rowBlockOffset[b + 1];
    if (t0 != tb0 || a.units[3ull * unit + 2] == tb1) return;  // not the first unit of a shared row block
    const std::uint32_t nu = (tb1 - tb0 + a.unitTiles - 1) / a.unitTiles;
    const unsigned r = threadIdx.x / 16, q = threadIdx.x % 16;
    const std::uint32_t f = slice * kSlice + 4 * q;
    const float* p = a.partials + (static_cast<std::uint64_t>(unit) * kTile + r) * a.ldh + f;
    const std::uint64_t stride = static_cast<std::uint64_t>(kTile) * a.ldh;
    constexpr std::uint32_t kIn = 8;
    f32x4 s[kIn];
#pragma unroll
    for (std::uint32_t j = 0; j < kIn; ++j) s[j] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    std::uint32_t k = 0;
    for (; k + kIn <= nu; k += kIn)
#pragma unroll
        for (std::uint32_t j = 0; j < kIn; ++j) s[j] += load_global<vf4>(p + (k + j) * stride);
    for (; k < nu; ++k) s[0] += load_global<vf4>(p + k * stride);
#pragma unroll
    for (std::uint32_t j = 1; j < kIn; ++j) s[0] += s[j];
    const bool vec = a.F % 4 == 0 && (reinterpret_cast<std::uintptr_t>(a.Y) & 15u) == 0;
    add_quad(y_row(a, b, r), f, a.F, vec, s[0]);
}

inline std::uint32_t hub_ldh(std::uint32_t F) { return (F + kSlice - 1) / kSlice * kSlice; }

}  // namespace
}  // namespace tcc

using namespace tcc;

extern "C" {

int tcc_hybrid_release(tcc_hybrid* H) {
    clear_last_error();
    if (!H) return TCC_OK;
    if (H->tilesAllocation) TCC_HIP_CHECK(hipFree(H->tilesAllocation));
    if (H->restAllocation) TCC_HIP_CHECK(hipFree(H->restAllocation));
    std::memset(H, 0, sizeof(*H));
    return TCC_OK;
}

int tcc_coo_to_hybrid(const std::uint32_t* dRow, const std::uint32_t* dCol, const float* dVal, std::uint32_t nnz,
                      std::uint32_t numRows, std::uint32_t numCols, std::uint32_t minTileNnz, std::uint32_t unitTiles,
                      std::uint32_t phases, tcc_hybrid* out, void* stream) {
    clear_last_error();
    TCC_REQUIRE(out && numRows >= 1 && numCols >= 1 && (nnz == 0 || (dRow && dCol)), TCC_ERR_INVALID_ARGUMENT,
                "invalid COO -> hybrid arguments");
    if (minTileNnz == 0) minTileNnz = kDefaultMinTileNnz;
    if (unitTiles == 0) unitTiles = kDefaultUnitTiles;
    TCC_REQUIRE(minTileNnz <= kTileVals, TCC_ERR_INVALID_ARGUMENT, "hybrid: minTileNnz above 256 leaves no tile");
    TCC_REQUIRE(unitTiles <= kMaxUnitTiles, TCC_ERR_INVALID_ARGUMENT, "hybrid: unitTiles above 64");
    const hipStream_t st = as_stream(stream);
    std::memset(out, 0, sizeof(*out));
    const std::uint32_t E = nnz;
    const std::uint32_t RB = (numRows + kTile - 1) / kTile;
    const std::uint32_t CB = (numCols + kTile - 1) / kTile;
    const std::uint64_t En = std::max<std::uint32_t>(E, 1);
    const std::uint64_t Vn = std::max<std::uint64_t>({En, numRows, numCols});
    const unsigned tileBits = std::max(1u, rank_bits(static_cast<std::uint64_t>(RB) * CB));
    TCC_REQUIRE(tileBits + 8 <= 64, TCC_ERR_UNSUPPORTED, "hybrid: tile key exceeds 64 bits");
    const std::uint64_t tempElems = std::max({radix_temp_elems(Vn), scan_temp_elems(En + 1),
                                              scan_temp_elems(static_cast<std::uint64_t>(RB) + 1)});

    std::uint64_t *keysA, *keysB;
    std::uint32_t *permA, *permB, *flags, *pos, *tileStart, *dense, *denseId, *restFlag, *restPos, *rowDeg, *colDeg,
        *rowRank, *colRank, *rowOrder, *colOrder, *blockTiles, *unitCount, *temp, *small, *restRow, *restCol;
    float* restVal;
    auto carve = [&](char* base) {
        std::size_t off = 0;
        auto take = [&](std::size_t bytes) {
            char* p = base ? base + off : nullptr;
            off += align_up(bytes);
            return p;
        };
        keysA = reinterpret_cast<std::uint64_t*>(take(8 * Vn));
        keysB = reinterpret_cast<std::uint64_t*>(take(8 * Vn));
        permA = reinterpret_cast<std::uint32_t*>(take(4 * En));
        permB = reinterpret_cast<std::uint32_t*>(take(4 * En));
        flags = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        pos = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        tileStart = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        dense = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        denseId = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        restFlag = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        restPos = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        rowDeg = reinterpret_cast<std::uint32_t*>(take(4 * (numRows + 1)));
        colDeg = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        rowRank = reinterpret_cast<std::uint32_t*>(take(4 * (numRows + 1)));
        colRank = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        rowOrder = reinterpret_cast<std::uint32_t*>(take(4ull * RB * kTile));
        colOrder = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        blockTiles = reinterpret_cast<std::uint32_t*>(take(4 * (RB + 1)));
        unitCount = reinterpret_cast<std::uint32_t*>(take(4 * (RB + 1)));
        restRow = reinterpret_cast<std::uint32_t*>(take(4 * En));
        restCol = reinterpret_cast<std::uint32_t*>(take(4 * En));
        restVal = reinterpret_cast<float*>(take(4 * En));
        temp = reinterpret_cast<std::uint32_t*>(take(4 * tempElems));
        small = reinterpret_cast<std::uint32_t*>(take(256));  // [0]=err [1]=tiles [2]=dense [3]=rest [4]=units [5]=hubBlocks
        return off;
    };
    const std::size_t scratchBytes = carve(nullptr);
    DevBuf<char> scratch;
    TCC_HIP_CHECK(hipMalloc(&scratch.p, scratchBytes));
    carve(scratch.p);

    TCC_HIP_CHECK(fill<std::uint32_t>(small, 64, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(rowDeg, numRows, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(colDeg, numCols, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(blockTiles, RB + 1, 0u, st));
    // dense[] is scanned over E entries; only the first (tile count) are set below
    TCC_HIP_CHECK(fill<std::uint32_t>(dense, En, 0u, st));
    TCC_HIP_CHECK(degree_histogram(dRow, E, numRows, rowDeg, small, st));
    TCC_HIP_CHECK(degree_histogram(dCol, E, numCols, colDeg, small, st));
    std::uint32_t hostSmall[8] = {};
    TCC_HIP_CHECK(hipMemcpyAsync(hostSmall, small, sizeof(hostSmall), hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    TCC_REQUIRE(hostSmall[0] == 0, TCC_ERR_INVALID_ARGUMENT, "COO index out of range");
    TCC_HIP_CHECK(degree_ranks(rowDeg, numRows, RB * kTile, rowRank, rowOrder, keysA, keysB, temp, st));
    TCC_HIP_CHECK(degree_ranks(colDeg, numCols, numCols, colRank, colOrder, keysA, keysB, temp, st));

    std::uint64_t* sorted = keysA;
    std::uint32_t* perm = permA;
    if (E > 0) {
        hipLaunchKernelGGL(tile_keys_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, dRow, dCol, E, rowRank,
                           colRank, CB, keysA, permA);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(radix_sort_pairs(keysA, keysB, permA, permB, E, tileBits + 8, temp, &sorted, &perm, st));
        hipLaunchKernelGGL(tile_heads_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, E, flags, small);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(flags, pos, E, small + 1, temp, st));
        hipLaunchKernelGGL(tile_start_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, flags, pos, E,
                           tileStart);
        hipLaunchKernelGGL(dense_tiles_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, tileStart,
                           small + 1, E, minTileNnz, CB, dense, blockTiles, small + 5);
        TCC_LAUNCH_CHECK();
        // dense ids over the E-sized flag array (zero past the tile count)
        TCC_HIP_CHECK(exclusive_scan(dense, denseId, E, small + 2, temp, st));
        hipLaunchKernelGGL(rest_flags_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, flags, pos, dense, E,
                           restFlag);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(restFlag, restPos, E, small + 3, temp, st));
    }
    hipLaunchKernelGGL(units_per_block_kernel, dim3(grid_for(RB, kThreads)), dim3(kThreads), 0, st, blockTiles, RB,
                       unitTiles, unitCount);
    TCC_LAUNCH_CHECK();
    TCC_HIP_CHECK(exclusive_scan(unitCount, unitCount, RB, small + 4, temp, st));
    TCC_HIP_CHECK(hipMemcpyAsync(hostSmall, small, sizeof(hostSmall), hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    TCC_REQUIRE(hostSmall[0] == 0, TCC_ERR_INVALID_ARGUMENT,
                hostSmall[0] == 2 ? "duplicate (row, col) entries in the COO input" : "COO index out of range");
    const std::uint32_t ND = E > 0 ? hostSmall[2] : 0;
    const std::uint32_t NR = E > 0 ? hostSmall[3] : 0;
    const std::uint32_t NU = hostSmall[4];
    const std::uint32_t hubCols = std::min(hostSmall[5] * kTile, numCols);

    // tiles part: rowOrder[16 RB] hubColOrder[hubCols] rowBlockOffset[RB+1] unitFirst[RB+1] tileCol[ND]
    // units[3 NU] tileVals[256 ND]
    const std::uint64_t NDn = std::max<std::uint32_t>(ND, 1);
    const std::size_t tilesBytes = align_up(4ull * RB * kTile) + align_up(4ull * std::max(hubCols, 1u)) +
                                   align_up(4ull * (RB + 1)) + align_up(4ull * (RB + 1)) + align_up(4 * NDn) +
                                   align_up(12ull * std::max(NU, 1u)) + align_up(4ull * kTileVals * NDn);
    char* o = nullptr;
    TCC_HIP_CHECK(hipMalloc(&o, tilesBytes));
    char* q = o;
    auto takeOut = [&](std::size_t bytes) {
        char* p = q;
        q += align_up(bytes);
        return p;
    };
    auto* oRowOrder = reinterpret_cast<std::uint32_t*>(takeOut(4ull * RB * kTile));
    auto* oHubCols = reinterpret_cast<std::uint32_t*>(takeOut(4ull * std::max(hubCols, 1u)));
    auto* oRowBlockOffset = reinterpret_cast<std::uint32_t*>(takeOut(4ull * (RB + 1)));
    auto* oUnitFirst = reinterpret_cast<std::uint32_t*>(takeOut(4ull * (RB + 1)));
    auto* oTileCol = reinterpret_cast<std::uint32_t*>(takeOut(4 * NDn));
    auto* oUnits = reinterpret_cast<std::uint32_t*>(takeOut(12ull * std::max(NU, 1u)));
    auto* oTileVals = reinterpret_cast<float*>(takeOut(4ull * kTileVals * NDn));
    auto fail = [&](int rc) {
        (void)hipFree(o);
        return rc;
    };
    if (hipMemcpyAsync(oRowOrder, rowOrder, 4ull * RB * kTile, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        (hubCols && hipMemcpyAsync(oHubCols, colOrder, 4ull * hubCols, hipMemcpyDeviceToDevice, st) != hipSuccess) ||
        exclusive_scan(blockTiles, oRowBlockOffset, RB, oRowBlockOffset + RB, temp, st) != hipSuccess ||
        hipMemcpyAsync(oUnitFirst, unitCount, 4ull * RB, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        hipMemcpyAsync(oUnitFirst + RB, small + 4, 4, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        fill<float>(oTileVals, kTileVals * NDn, 0.0f, st) != hipSuccess) {
        set_last_error("HIP error while initialising the hub tiles");
        return fail(TCC_ERR_HIP);
    }
    if (E > 0) {
        hipLaunchKernelGGL(place_entries_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, perm, E,
                           flags, pos, dense, denseId, restPos, dRow, dCol, dVal, oTileVals, restRow, restCol,
                           dVal ? restVal : nullptr);
        hipLaunchKernelGGL(tile_cols_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, tileStart,
                           small + 1, dense, denseId, CB, oTileCol);
    }
    hipLaunchKernelGGL(tile_units_kernel, dim3(grid_for(RB, kThreads)), dim3(kThreads), 0, st, oRowBlockOffset,
                       oUnitFirst, RB, unitTiles, oUnits);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        set_last_error("HIP error while building the hub tiles");
        return fail(TCC_ERR_HIP);
    }
    // the remainder: an ordinary or phased BCSR of the entries outside dense tiles
    tcc_bcsr rest{};
    void* restAlloc = nullptr;
    const int rc = tcc_coo_to_bcsr_phased(NR ? restRow : nullptr, NR ? restCol : nullptr, dVal ? restVal : nullptr, NR,
                                          numRows, numCols, phases, &rest, &restAlloc, stream);
    if (rc) return fail(rc);

    tcc_hub_tiles& T = out->tiles;
    T.num_rows = numRows;
    T.num_cols = numCols;
    T.nnz = E - NR;
    T.num_row_blocks = RB;
    T.num_tiles = ND;
    T.num_units = NU;
    T.unit_tiles = unitTiles;
    T.hub_cols = hubCols;
    T.rowOrder = oRowOrder;
    T.hubColOrder = oHubCols;
    T.rowBlockOffset = oRowBlockOffset;
    T.tileCol = oTileCol;
    T.tileVals = oTileVals;
    T.units = oUnits;
    out->rest = rest;
    out->tilesAllocation = o;
    out->restAllocation = restAlloc;
    return TCC_OK;
}

size_t tcc_hybrid_workspace_bytes(const tcc_hybrid* H, std::uint32_t featureDim) {
    if (!H || featureDim == 0) return 0;
    return align_up(tcc_tf32_packed_bytes(H->rest.num_cols, featureDim) + 16) +
           tcc_hub_tiles_workspace_bytes(&H->tiles, featureDim);
}

size_t tcc_hub_tiles_workspace_bytes(const tcc_hub_tiles* T, std::uint32_t featureDim) {
    if (!T || featureDim == 0) return 0;
    const std::size_t ldh = hub_ldh(featureDim);
    return align_up(static_cast<size_t>(T->hub_cols) * ldh * sizeof(float)) +
           static_cast<size_t>(T->num_units) * kTile * ldh * sizeof(float);
}

int tcc_hub_tiles_spmm(const tcc_hub_tiles* T, const float* X, float* Y, std::uint32_t featureDim, void* workspace,
                       size_t workspaceBytes, void* stream) {
    clear_last_error();
    TCC_REQUIRE(T && X && Y && featureDim >= 1 && T->rowOrder && T->rowBlockOffset, TCC_ERR_INVALID_ARGUMENT,
                "invalid hub tiles SpMM arguments");
    if (T->num_units == 0) return TCC_OK;
    TCC_REQUIRE(T->tileCol && T->tileVals && T->units && T->hubColOrder, TCC_ERR_INVALID_ARGUMENT,
                "invalid hub tiles SpMM arguments");
    TCC_REQUIRE(T->unit_tiles >= 1 && T->unit_tiles <= kMaxUnitTiles, TCC_ERR_INVALID_ARGUMENT,
                "hub tiles: unit_tiles must be 1..64");
    const std::uint32_t ldh = hub_ldh(featureDim);
    TCC_REQUIRE(workspace && workspaceBytes >= tcc_hub_tiles_workspace_bytes(T, featureDim) &&
                    reinterpret_cast<std::uintptr_t>(workspace) % 16 == 0,
                TCC_ERR_INVALID_ARGUMENT, "hub tiles SpMM workspace too small or misaligned");
    const hipStream_t st = as_stream(stream);
    float* Xh = static_cast<float*>(workspace);
    const std::uint64_t n = static_cast<std::uint64_t>(T->hub_cols) * ldh;
    hipLaunchKernelGGL(hub_rows_kernel, dim3(grid_for(n, kThreads)), dim3(kThreads), 0, st, X, featureDim,
                       T->hubColOrder, T->hub_cols, ldh, Xh);
    TCC_LAUNCH_CHECK();
    TileArgs a{};
    a.rowOrder = T->rowOrder;
    a.rowBlockOffset = T->rowBlockOffset;
    a.tileCol = T->tileCol;
    a.tileVals = T->tileVals;
    a.units = T->units;
    a.Xh = Xh;
    a.ldh = ldh;
    a.Y = Y;
    a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(n * sizeof(float)));
    a.F = featureDim;
    a.numUnits = T->num_units;
    a.slices = ldh / kSlice;
    a.unitTiles = T->unit_tiles;
    const std::uint64_t waves = static_cast<std::uint64_t>(a.numUnits) * a.slices;
    TCC_REQUIRE(waves <= 0x7FFFFFFFull, TCC_ERR_UNSUPPORTED, "hub tiles SpMM launch too large");
    hipLaunchKernelGGL(hub_tiles_kernel<kStages>, dim3(grid_for(waves, kThreads / kWave)), dim3(kThreads), 0, st, a);
    TCC_LAUNCH_CHECK();
    hipLaunchKernelGGL(hub_reduce_kernel, dim3(static_cast<std::uint32_t>(waves)), dim3(kThreads), 0, st, a);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

int tcc_hybrid_spmm(const tcc_hybrid* H, const float* X, float* Y, std::uint32_t featureDim, int accumulate,
                    void* workspace, size_t workspaceBytes, void* stream) {
    clear_last_error();
    TCC_REQUIRE(H && X && Y && featureDim >= 1 && workspace, TCC_ERR_INVALID_ARGUMENT, "invalid hybrid SpMM arguments");
    TCC_REQUIRE(workspaceBytes >= tcc_hybrid_workspace_bytes(H, featureDim) &&
                    reinterpret_cast<std::uintptr_t>(workspace) % 16 == 0,
                TCC_ERR_INVALID_ARGUMENT, "hybrid SpMM workspace too small or misaligned (tcc_hybrid_workspace_bytes)");
    // The remainder's product writes (or adds into) Y, over packed TF32 rows
    // when its rows are gathered often (8 blocks per column on average,
    // 16 gathers per row), else over X; then the tiles add theirs.
    const std::uint64_t gathers = 8ull * H->rest.num_TCBlocks;
    const std::size_t packedBytes = align_up(tcc_tf32_packed_bytes(H->rest.num_cols, featureDim) + 16);
    int rc;
    if (gathers >= 16ull * H->rest.num_cols) {
        rc = tcc_tf32_pack(X, H->rest.num_cols, featureDim, workspace, stream);
        if (rc) return rc;
        rc = tcc_bcsr_spmm_packed(&H->rest, workspace, Y, featureDim, accumulate, stream);
    } else {
        rc = tcc_bcsr_spmm(&H->rest, X, Y, featureDim, accumulate, stream);
    }
    if (rc) return rc;
    return tcc_hub_tiles_spmm(&H->tiles, X, Y, featureDim, static_cast<char*>(workspace) + packedBytes,
                              workspaceBytes - packedBytes, stream);
}

}  // extern "C"
