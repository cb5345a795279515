// Row super-window BCSR on gfx950: construction and the SpMM over packed
// TF32 feature rows (no reference counterpart; the product is the one
// tf32_spmm_bcsr computes, spmm_cnic/src/core/spmm_kernel.cu:1560-1842).
//
// Format.  Rows are ordered by degree (descending, ties by row id) and cut
// into super-windows of 64 rows, 8 row windows of 8.  Each super-window lists
// the distinct source columns its rows use (ordered by the columns' own
// degree rank, hub columns first), one (super-window, column) "pair" each,
// with a 64-bit mask: bit 8w+r = row r of window w uses the column.  The
// values follow pair by pair in mask-bit order, so the values of window w in
// pair p start at pairValue[p] + popcount(mask & (2^{8w} - 1)).
//
// Why.  On skewed (R-MAT) graphs the rows of a degree-sorted super-window
// share most of their columns: at the 233k-node, 114M-nnz configuration an
// 8-row window of the ordinary BCSR holds 102.9M (window, column) pairs, 1.1
// nonzeros each, and every one of them loads its feature row; degree-sorted
// super-windows of 64 rows hold 32.7M pairs.  A workgroup takes one unit of
// a super-window (a run of its pairs, one 256-feature chunk), stages the
// packed feature rows of TP pairs at a time in LDS (double-buffered), and
// each of its 8 waves accumulates its own row window from LDS, so a feature
// row is fetched once per pair, not once per (window, column).  Rows of
// similar degree also give the 8 waves similar work between barriers.
//
// Output rows go back to their original positions (rowOrder).  A
// super-window cut into several units has its rows zeroed first (unless
// accumulating) and receives each unit's partial sums with fp32 atomics;
// a super-window held by one unit is stored directly.
#include <algorithm>
#include <cstring>

#include "../../include/tcc_spmm_cnic.h"
#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "degree_rank.hpp"
#include "primitives.hpp"

namespace tcc {
namespace {

constexpr unsigned kSwRows = 64;         // rows per super-window
constexpr unsigned kSwWaves = kSwRows / 8;  // one wave per row window
constexpr unsigned kSwThreads = kSwWaves * kWave;
constexpr std::uint32_t kSwDefaultUnitPairs = 2048;
constexpr std::uint32_t kSwMaxPhases = 16;
constexpr std::uint32_t kPackChunkF = 256;      // features per packed chunk (tcc_tf32_pack)
constexpr std::uint32_t kPackChunkB = 640;      // bytes of a full packed chunk
constexpr unsigned kBuildThreads = 256;

inline unsigned ceil_log2(std::uint64_t x) {
    unsigned b = 0;
    while ((1ull << b) < x) ++b;
    return b;
}

inline std::size_t align_up(std::size_t x) { return (x + 255) & ~std::size_t(255); }

__host__ __device__ constexpr std::uint32_t packed_chunk_bytes(std::uint32_t n) {
    return n >= kPackChunkF ? kPackChunkB : static_cast<std::uint32_t>(((2ull * n + (n + 1) / 2) + 15) & ~15ull);
}

__host__ __device__ constexpr std::uint64_t packed_row_stride(std::uint32_t F) {
    const std::uint64_t full = F / kPackChunkF, tail = F % kPackChunkF;
    const std::uint64_t bytes = full * kPackChunkB + (tail ? packed_chunk_bytes(static_cast<std::uint32_t>(tail)) : 0);
    return F > kPackChunkF ? ((bytes + 127) & ~127ull) : bytes;
}

// ---------------------------------------------------------------- builder

// Edge key (super-window, column rank, row in super-window); payload = edge.
__global__ void sw_keys_kernel(const std::uint32_t* __restrict__ row, const std::uint32_t* __restrict__ col,
                               std::uint32_t E, const std::uint32_t* __restrict__ rowRank,
                               const std::uint32_t* __restrict__ colRank, unsigned colBits,
                               std::uint64_t* __restrict__ keys, std::uint32_t* __restrict__ perm) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint32_t rr = rowRank[row[e]];
    const std::uint64_t g = rr / kSwRows;
    keys[e] = (((g << colBits) | colRank[col[e]]) << 6) | (rr % kSwRows);
    perm[e] = e;
}

// Pair heads; a repeated full key is a duplicate edge.
__global__ void sw_flags_kernel(const std::uint64_t* __restrict__ keys, std::uint32_t E, unsigned colBits,
                                std::uint32_t* __restrict__ flags, std::uint32_t* __restrict__ groupPairs,
                                std::uint32_t* __restrict__ err) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint64_t k = keys[e];
    const bool head = e == 0 || (k >> 6) != (keys[e - 1] >> 6);
    if (e > 0 && k == keys[e - 1]) atomicMax(err, 2u);
    flags[e] = head ? 1u : 0u;
    if (head) aggregated_increment(groupPairs, static_cast<std::uint32_t>(k >> (colBits + 6)));
}

// Pairs per column rank (to place the phase boundaries).
__global__ void rank_pairs_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ flags,
                                  std::uint32_t E, std::uint64_t colMask, std::uint32_t* __restrict__ rankPairs) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < E && flags[e]) atomicAdd(&rankPairs[static_cast<std::uint32_t>((keys[e] >> 6) & colMask)], 1u);
}

// Phase k (1 <= k < phases) starts at the first column rank r whose earlier
// ranks hold at least ceil(k * pairs / phases) pairs (bounds preset to
// numCols: an empty phase).
__global__ void phase_bounds_kernel(const std::uint32_t* __restrict__ cumExcl, std::uint32_t numCols,
                                    const std::uint32_t* __restrict__ total, std::uint32_t phases,
                                    std::uint32_t* __restrict__ bounds) {
    const std::uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= numCols) return;
    const std::uint32_t totalPairs = *total;
    for (std::uint32_t k = 1; k < phases; ++k) {
        const std::uint64_t t = (static_cast<std::uint64_t>(k) * totalPairs + phases - 1) / phases;
        if (t > 0 && cumExcl[r] >= t && (r == 0 || cumExcl[r - 1] < t)) bounds[k] = r;
    }
}

__device__ __forceinline__ std::uint32_t phase_of(std::uint32_t rank, const std::uint32_t* bounds,
                                                  std::uint32_t phases) {
    std::uint32_t ph = 0;
    for (std::uint32_t k = 1; k < phases; ++k) ph += rank >= bounds[k] ? 1u : 0u;
    return ph;
}

// Pairs per (phase, super-window), index phase * G + g.
__global__ void phase_counts_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ flags,
                                    std::uint32_t E, unsigned colBits, const std::uint32_t* __restrict__ bounds,
                                    std::uint32_t phases, std::uint32_t G, std::uint32_t* __restrict__ counts) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E || !flags[e]) return;
    const std::uint64_t k = keys[e] >> 6;
    const std::uint32_t rank = static_cast<std::uint32_t>(k & ((1ull << colBits) - 1ull));
    const std::uint32_t g = static_cast<std::uint32_t>(k >> colBits);
    atomicAdd(&counts[phase_of(rank, bounds, phases) * G + g], 1u);
}

// Units per (phase, super-window); a super-window without pairs keeps one
// (empty) unit in phase 0, which stores its zero rows.
__global__ void phase_units_kernel(const std::uint32_t* __restrict__ counts, const std::uint32_t* __restrict__ groupPairs,
                                   std::uint32_t G, std::uint32_t phases, std::uint32_t unitPairs,
                                   std::uint32_t* __restrict__ units) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= G * phases) return;
    const std::uint32_t g = i % G;
    std::uint32_t u = (counts[i] + unitPairs - 1) / unitPairs;
    if (i < G && groupPairs[g] == 0) u = 1;
    units[i] = u;
}

// Pair columns, masks and value offsets (the sorted position of the pair's
// first edge: values are stored in sorted-edge order), and the values.
__global__ void sw_place_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ perm,
                                std::uint32_t E, const std::uint32_t* __restrict__ flags,
                                const std::uint32_t* __restrict__ pos, const std::uint32_t* __restrict__ col,
                                const float* __restrict__ val, std::uint32_t* __restrict__ pairCol,
                                unsigned long long* __restrict__ pairMask, std::uint32_t* __restrict__ pairValue,
                                float* __restrict__ data) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint64_t k = keys[e];
    const std::uint32_t p = pos[e] + flags[e] - 1;
    const std::uint32_t src = perm[e];
    if (flags[e]) {
        pairCol[p] = col[src];
        pairValue[p] = e;
    }
    atomicOr(&pairMask[p], 1ull << (k & 63u));
    if (data) data[e] = val ? val[src] : 1.0f;
}

// units[3u .. 3u+2] = super-window, first pair, end pair of unit u; units
// are ordered phase first, then super-window.
__global__ void sw_units_kernel(const std::uint32_t* __restrict__ groupOffset, const std::uint32_t* __restrict__ counts,
                                const std::uint32_t* __restrict__ unitFirst, std::uint32_t G, std::uint32_t phases,
                                std::uint32_t unitPairs, std::uint32_t* __restrict__ units) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= G * phases) return;
    const std::uint32_t g = i % G, ph = i / G;
    std::uint32_t start = groupOffset[g];
    for (std::uint32_t q = 0; q < ph; ++q) start += counts[q * G + g];
    const std::uint32_t end = start + counts[i];
    const std::uint32_t n = unitFirst[i + 1] - unitFirst[i];
    for (std::uint32_t k = 0; k < n; ++k) {
        const std::uint64_t u = 3ull * (unitFirst[i] + k);
        units[u] = g;
        units[u + 1] = start + k * unitPairs;
        units[u + 2] = min(start + (k + 1) * unitPairs, end);
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

struct SwArgs {
    const std::uint32_t* rowOrder;
    const std::uint32_t* groupOffset;
    const std::uint32_t* pairCol;
    const std::uint64_t* pairMask;
    const std::uint32_t* pairValue;
    const float* data;
    const std::uint32_t* units;
    const unsigned char* packed;
    std::uint64_t stride;  // bytes per packed row
    float* Y;
    std::uint32_t F;
    std::uint32_t numUnits;
    std::uint32_t numChunks;
    int accumulate;
};

// Zero the rows of every super-window cut into more than one unit (they
// receive atomics): the unit holding its first pair does it.  One
// workgroup per unit.
__global__ void __launch_bounds__(256) sw_zero_shared_kernel(SwArgs a) {
    const std::uint32_t u = blockIdx.x;
    const std::uint32_t g = a.units[3ull * u];
    const std::uint32_t gBeg = a.groupOffset[g], gEnd = a.groupOffset[g + 1];
    if (a.units[3ull * u + 1] != gBeg || a.units[3ull * u + 2] == gEnd) return;
    for (unsigned r = 0; r < kSwRows; ++r) {
        const std::uint32_t orow = a.rowOrder[g * kSwRows + r];
        if (orow == TCC_SWTCF_INVALID_ROW_SLOT) continue;
        float* p = a.Y + static_cast<std::uint64_t>(orow) * a.F;
        for (std::uint32_t f = threadIdx.x; f < a.F; f += blockDim.x) p[f] = 0.0f;
    }
}

// Lane-uniform byte of a 64-bit mask held as two halves.
__device__ __forceinline__ std::uint32_t wave_byte(std::uint32_t lo, std::uint32_t hi, unsigned w) {
    return ((w < 4 ? lo : hi) >> (8 * (w & 3u))) & 0xFFu;
}

// One workgroup of 8 waves per (unit, 256-feature chunk), chunk-major.  Wave
// w owns row window w of the unit's super-window; lane l holds features
// 4l..4l+3 of the chunk for its 8 rows.  TP pairs per LDS stage.
template <int TP, bool VALUES>
__global__ void __launch_bounds__(kSwThreads) sw_gather_kernel(SwArgs a) {
    static_assert(TP == 16 || TP == 32 || TP == 64, "pairs per stage");
    constexpr unsigned kPieces = TP * kPackChunkB / 16;  // 16-byte pieces of a full stage
    constexpr unsigned kLoads = (kPieces + kSwThreads - 1) / kSwThreads;
    constexpr unsigned kSub = TP / 8;  // 8-pair value groups per stage
    __shared__ __attribute__((aligned(16))) unsigned char stage[2][TP * kPackChunkB];

    const unsigned lane = __lane_id();
    const unsigned wave = static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave)));
    const std::uint32_t chunk = blockIdx.x / a.numUnits;
    const std::uint32_t unit = blockIdx.x - chunk * a.numUnits;
    const std::uint32_t g = a.units[3ull * unit];
    const std::uint32_t p0 = a.units[3ull * unit + 1];
    const std::uint32_t p1 = a.units[3ull * unit + 2];
    const std::uint32_t gBeg = a.groupOffset[g], gEnd = a.groupOffset[g + 1];
    const bool shared = p0 != gBeg || p1 != gEnd;
    const std::uint32_t fBase = chunk * kPackChunkF;
    const std::uint32_t n = min(kPackChunkF, a.F - fBase);  // features of this chunk
    const std::uint32_t cb = packed_chunk_bytes(n);         // staged bytes per pair
    const std::uint32_t cp = cb / 16;                       // 16-byte pieces per pair
    const bool active = 4 * lane < n;
    const std::uint32_t hiOff = active ? 8 * lane : 0;      // the lane's 4 high halves
    const std::uint32_t loOff = active ? 2 * n + 2 * lane : 0;  // and their low bits
    const std::uint64_t chunkOff = static_cast<std::uint64_t>(chunk) * kPackChunkB;
    // The 16-byte pieces this thread stages: piece j = tid + i*threads is
    // byte 16*j of the stage, pair j / cp, byte 16*(j % cp) of its row chunk
    // (the same for every stage).
    std::uint32_t pieceT[kLoads], pieceSrc[kLoads];
#pragma unroll
    for (unsigned i = 0; i < kLoads; ++i) {
        const std::uint32_t j = threadIdx.x + i * kSwThreads;
        pieceT[i] = j / cp;
        pieceSrc[i] = 16 * (j - pieceT[i] * cp);
    }

    float acc[8][4];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[r][j] = 0.0f;
    std::uint32_t touched = 0;

    // Loads complete in order, so anything computed from a load must wait
    // for every load issued before it.  Loaded data is therefore used only
    // an iteration or more after it was requested, and each iteration issues
    // its loads in the order they will be needed: the metadata of stage
    // k+3, the values of stage k+1, then the feature rows of stage k+2.
    // Waiting for the first two never waits for rows still in flight.

    // Stage metadata as loaded: lane l < TP holds pair p+l (clamped into the
    // unit; pairs past it are masked out when the metadata is used).
    struct Meta {
        std::uint32_t col, lo, hi, voff;
    };
    const std::uint32_t lastPair = p1 > p0 ? p1 - 1 : p0;
    auto load_meta = [&](std::uint32_t p) {
        Meta m;
        const std::uint32_t q = min(p + min(lane, static_cast<unsigned>(TP) - 1u), lastPair);
        m.col = a.pairCol[q];
        const vu2 mk = load_global<vu2>(a.pairMask + q);
        m.lo = mk.x;
        m.hi = mk.y;
        m.voff = VALUES ? a.pairValue[q] : 0u;
        return m;
    };
    // What this wave takes from a stage's metadata: its row byte of each
    // pair (zero for pairs outside the stage) and the offset of its first
    // value in each pair.
    struct Use {
        std::uint32_t mb, vb;
    };
    auto use_of = [&](const Meta& m, std::uint32_t p) {
        Use u;
        const bool valid = lane < static_cast<unsigned>(TP) && p + lane < p1;
        u.mb = valid ? wave_byte(m.lo, m.hi, wave) : 0u;
        const std::uint64_t mk = static_cast<std::uint64_t>(m.hi) << 32 | m.lo;
        const std::uint64_t below = wave == 0 ? 0ull : (mk & ((1ull << (8 * wave)) - 1ull));
        u.vb = m.voff + static_cast<std::uint32_t>(__popcll(below));
        return u;
    };
    // The stage's feature rows, kLoads 16-byte pieces per thread.
    struct Pieces {
        vu4 v[kLoads];
    };
    auto stage_count = [&](std::uint32_t p) { return p < p1 ? min(static_cast<std::uint32_t>(TP), p1 - p) : 0u; };
    auto issue_stage = [&](const Meta& m, std::uint32_t p, Pieces& pc) {
        const std::uint32_t count = stage_count(p);
        const unsigned char* base = a.packed + chunkOff;
#pragma unroll
        for (unsigned i = 0; i < kLoads; ++i) {
            const std::uint32_t c = static_cast<std::uint32_t>(
                __shfl(static_cast<int>(m.col), static_cast<int>(pieceT[i] & (kWave - 1))));
            if (pieceT[i] < count) pc.v[i] = load_global<vu4>(base + static_cast<std::uint64_t>(c) * a.stride + pieceSrc[i]);
        }
    };
    auto write_stage = [&](unsigned char* buf, std::uint32_t p, const Pieces& pc) {
        const std::uint32_t count = stage_count(p);
#pragma unroll
        for (unsigned i = 0; i < kLoads; ++i)
            if (pieceT[i] < count) *reinterpret_cast<vu4*>(buf + 16 * (threadIdx.x + i * kSwThreads)) = pc.v[i];
    };
    // Values of this wave's rows in the stage, as loaded: value group s,
    // lane 8k+r = pair 8s+k, row r (lanes whose row does not use the pair
    // read the pair's first value and are never read back).
    struct Vals {
        float v[kSub];
    };
    auto load_vals = [&](const Use& u) {
        Vals vs;
        const unsigned r = lane & 7u;
#pragma unroll
        for (unsigned s = 0; s < kSub; ++s) {
            const int t = static_cast<int>(8 * s + (lane >> 3));
            const std::uint32_t mt = static_cast<std::uint32_t>(__shfl(static_cast<int>(u.mb), t));
            const std::uint32_t vt = static_cast<std::uint32_t>(__shfl(static_cast<int>(u.vb), t));
            const std::uint32_t rank = ((mt >> r) & 1u) ? static_cast<std::uint32_t>(__popc(mt & ((1u << r) - 1u))) : 0u;
            vs.v[s] = a.data[vt + rank];
        }
        return vs;
    };

    // Add up the stage: the pairs this wave's rows use, value group by value
    // group (so that each group's value register is named statically), the
    // next pair's LDS reads issued before the current pair is added.
    auto compute = [&](const unsigned char* buf, const Use& u, const Vals& vs) {
        const std::uint32_t mb = u.mb;
        const std::uint64_t used = __ballot(mb != 0u);
        if (!used) return;
        auto read = [&](unsigned t, std::uint64_t& h, std::uint32_t& l) {
            const unsigned char* b = buf + t * cb;
            h = *reinterpret_cast<const std::uint64_t*>(b + hiOff);
            l = *reinterpret_cast<const std::uint16_t*>(b + loOff);
        };
#pragma unroll
        for (unsigned s = 0; s < kSub; ++s) {
            std::uint32_t us = static_cast<std::uint32_t>(used >> (8 * s)) & 0xFFu;
            if (!us) continue;
            // the forward products' values are TF32-rounded
            const float vv = VALUES ? tf32_rna(vs.v[s]) : 0.0f;
            std::uint64_t nh;
            std::uint32_t nl;
            read(8 * s + static_cast<unsigned>(__builtin_ctz(us)), nh, nl);
            while (us) {
                const unsigned k = static_cast<unsigned>(__builtin_ctz(us));
                us &= us - 1;
                const std::uint64_t h = nh;
                const std::uint32_t l = nl;
                if (us) read(8 * s + static_cast<unsigned>(__builtin_ctz(us)), nh, nl);
                const std::uint32_t mt = static_cast<std::uint32_t>(
                    __builtin_amdgcn_readlane(static_cast<int>(mb), static_cast<int>(8 * s + k)));
                touched |= mt;
                float x[4];
                const std::uint32_t h0 = static_cast<std::uint32_t>(h), h1 = static_cast<std::uint32_t>(h >> 32);
                x[0] = __uint_as_float((h0 << 16) | ((l & 7u) << 13));
                x[1] = __uint_as_float((h0 & 0xFFFF0000u) | (((l >> 3) & 7u) << 13));
                x[2] = __uint_as_float((h1 << 16) | (((l >> 8) & 7u) << 13));
                x[3] = __uint_as_float((h1 & 0xFFFF0000u) | (((l >> 11) & 7u) << 13));
                const int lb = static_cast<int>(k * 8);
                auto add_row = [&](int r) {
                    if constexpr (VALUES) {
                        const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vv), lb + r));
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[r][j] = fmaf(w, x[j], acc[r][j]);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) acc[r][j] += x[j];
                    }
                };
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    if ((mt >> r) & 1u) add_row(r);
            }
        }
    };

    // Stage k sits in LDS buffer k & 1 while the feature rows of stages k+1
    // and k+2 are in flight in registers (about 2 x TP x 640 bytes per
    // workgroup); one barrier per stage.
    const std::uint32_t stages = (p1 - p0 + TP - 1) / TP;
    if (stages > 0) {
        Meta m0 = load_meta(p0), m1 = load_meta(p0 + TP), m2 = load_meta(p0 + 2 * TP);
        Pieces pa, pb;
        issue_stage(m0, p0, pa);
        issue_stage(m1, p0 + TP, pb);
        Use u0 = use_of(m0, p0);
        Vals v0{};
        if constexpr (VALUES) v0 = load_vals(u0);
        write_stage(stage[0], p0, pa);
        __syncthreads();
        // Iteration k: `next` holds the rows of stage k+1, `free` receives
        // those of stage k+2.
        auto step = [&](std::uint32_t k, Pieces& next, Pieces& free) {
            const std::uint32_t p = p0 + k * TP;
            const Use u1 = use_of(m1, p + TP);
            const Meta m3 = load_meta(p + 3 * TP);
            Vals v1{};
            if constexpr (VALUES) v1 = load_vals(u1);
            issue_stage(m2, p + 2 * TP, free);
            compute(stage[k & 1], u0, v0);
            if (k + 1 < stages) write_stage(stage[(k + 1) & 1], p + TP, next);
            __syncthreads();
            u0 = u1;
            v0 = v1;
            m1 = m2;
            m2 = m3;
        };
        // Two steps per trip keep the register roles fixed; a step past the
        // last stage loads no rows and finds no pair in use.
        for (std::uint32_t k = 0; k < stages; k += 2) {
            step(k, pb, pa);
            step(k + 1, pa, pb);
        }
    }

    // Output rows of this wave's window (lane r < 8).
    std::uint32_t orow = TCC_SWTCF_INVALID_ROW_SLOT;
    if (lane < 8) orow = a.rowOrder[static_cast<std::uint64_t>(g) * kSwRows + wave * 8 + lane];
    const std::uint32_t fLane = fBase + 4 * lane;
    if (!shared) {
        const bool vec = (a.F % 4 == 0) && ((reinterpret_cast<std::uintptr_t>(a.Y) & 15u) == 0);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const std::uint32_t o = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(orow), r));
            if (o == TCC_SWTCF_INVALID_ROW_SLOT || !active) continue;
            float* out = a.Y + static_cast<std::uint64_t>(o) * a.F + fLane;
            if (vec && fLane + 3 < a.F) {
                float4 s = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
                if (a.accumulate) {
                    const float4 prev = *reinterpret_cast<const float4*>(out);
                    s.x += prev.x;
                    s.y += prev.y;
                    s.z += prev.z;
                    s.w += prev.w;
                }
                *reinterpret_cast<float4*>(out) = s;
            } else {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    if (fLane + j < a.F) out[j] = a.accumulate ? out[j] + acc[r][j] : acc[r][j];
            }
        }
        return;
    }
    // Shared super-window: each row's 256 sums pass through LDS so that
    // atomic instruction j adds features 64j..64j+63 of the chunk (one per
    // lane, 256 contiguous bytes) rather than every 4th float of 1 KB.
    // The stage buffers are free after the last barrier above.
    float* st = reinterpret_cast<float*>(stage[0]) + wave * (kWave * 4);
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const std::uint32_t o = static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(orow), r));
        if (!((touched >> r) & 1u) || o == TCC_SWTCF_INVALID_ROW_SLOT) continue;
        *reinterpret_cast<float4*>(st + 4 * lane) = make_float4(acc[r][0], acc[r][1], acc[r][2], acc[r][3]);
        __builtin_amdgcn_wave_barrier();
        float t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = st[kWave * j + lane];
        __builtin_amdgcn_wave_barrier();
        float* rb = a.Y + static_cast<std::uint64_t>(o) * a.F + fBase;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (kWave * j + lane < n) atomic_add_f32(rb + kWave * j + lane, t[j]);
    }
}

bool sw_ok(const tcc_sw_bcsr* A) {
    return A && A->num_groups >= 1 && A->num_units >= A->num_groups && A->unit_pairs >= 1 && A->rowOrder &&
           A->groupOffset && A->units && (A->num_pairs == 0 || (A->pairCol && A->pairMask)) &&
           (A->data == nullptr || A->pairValue != nullptr);
}

}  // namespace
}  // namespace tcc

using namespace tcc;

extern "C" {

int tcc_coo_to_sw_bcsr(const std::uint32_t* dRow, const std::uint32_t* dCol, const float* dVal, std::uint32_t nnz,
                       std::uint32_t numRows, std::uint32_t numCols, std::uint32_t unitPairs, std::uint32_t phases,
                       tcc_sw_bcsr* out, void** allocation, void* stream) {
    clear_last_error();
    TCC_REQUIRE(out && allocation && numRows >= 1 && numCols >= 1 && (nnz == 0 || (dRow && dCol)),
                TCC_ERR_INVALID_ARGUMENT, "invalid COO -> super-window BCSR arguments");
    if (unitPairs == 0) unitPairs = kSwDefaultUnitPairs;
    if (phases == 0) phases = 1;
    TCC_REQUIRE(phases <= kSwMaxPhases, TCC_ERR_INVALID_ARGUMENT, "super-window BCSR: at most 16 phases");
    const hipStream_t st = as_stream(stream);
    std::memset(out, 0, sizeof(*out));
    *allocation = nullptr;
    const std::uint32_t E = nnz;
    const std::uint32_t G = (numRows + kSwRows - 1) / kSwRows;
    const std::uint32_t padded = G * kSwRows;
    const unsigned rowBits = std::max(1u, ceil_log2(numRows));
    const unsigned colBits = std::max(1u, ceil_log2(numCols));
    const unsigned groupBits = std::max(1u, ceil_log2(G));
    TCC_REQUIRE(groupBits + colBits + 6 <= 64, TCC_ERR_UNSUPPORTED, "super-window key exceeds 64 bits");

    // scratch
    const std::uint64_t En = std::max<std::uint32_t>(E, 1);
    const std::uint64_t Vn = std::max<std::uint64_t>({En, numRows, numCols});
    const std::uint64_t GP = static_cast<std::uint64_t>(G) * phases;
    const std::uint64_t tempElems = std::max({radix_temp_elems(Vn), scan_temp_elems(En + 1), scan_temp_elems(GP + 1),
                                              scan_temp_elems(static_cast<std::uint64_t>(numCols) + 1)});
    std::uint64_t *keysA, *keysB;
    std::uint32_t *permA, *permB, *flags, *pos, *rowDeg, *colDeg, *rowRank, *colRank, *groupPairs, *unitCount, *temp,
        *small, *rankPairs, *rankCum, *phaseCounts, *bounds;
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
        rowDeg = reinterpret_cast<std::uint32_t*>(take(4 * (numRows + 1)));
        colDeg = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        rowRank = reinterpret_cast<std::uint32_t*>(take(4 * (numRows + 1)));
        colRank = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        groupPairs = reinterpret_cast<std::uint32_t*>(take(4 * (G + 1)));
        unitCount = reinterpret_cast<std::uint32_t*>(take(4 * (GP + 1)));
        rankPairs = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        rankCum = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        phaseCounts = reinterpret_cast<std::uint32_t*>(take(4 * (GP + 1)));
        bounds = reinterpret_cast<std::uint32_t*>(take(4 * kSwMaxPhases));
        temp = reinterpret_cast<std::uint32_t*>(take(4 * tempElems));
        small = reinterpret_cast<std::uint32_t*>(take(256));  // [0]=err [1]=pairs [2]=units
        return off;
    };
    const std::size_t scratchBytes = carve(nullptr);
    DevBuf<char> scratch;
    TCC_HIP_CHECK(hipMalloc(&scratch.p, scratchBytes));
    carve(scratch.p);

    // outputs whose size is known now: rowOrder[64G], groupOffset[G+1]
    TCC_HIP_CHECK(fill<std::uint32_t>(small, 64, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(rowDeg, numRows, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(colDeg, numCols, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(groupPairs, G + 1, 0u, st));
    DevBuf<std::uint32_t> rowOrderTmp;
    TCC_HIP_CHECK(hipMalloc(&rowOrderTmp.p, 4ull * padded));
    if (E > 0) {
        TCC_HIP_CHECK(degree_histogram(dRow, E, numRows, rowDeg, small, st));
        TCC_HIP_CHECK(degree_histogram(dCol, E, numCols, colDeg, small, st));
    }
    // row and column ranks: degree descending, ids ascending
    TCC_HIP_CHECK(degree_ranks(rowDeg, numRows, padded, rowRank, rowOrderTmp.p, keysA, keysB, temp, st));
    TCC_HIP_CHECK(degree_ranks(colDeg, numCols, numCols, colRank, nullptr, keysA, keysB, temp, st));

    // Error check before the edge keys read the ranks of their indices.
    std::uint32_t hostSmall[4] = {0, 0, 0, 0};
    TCC_HIP_CHECK(hipMemcpyAsync(hostSmall, small, sizeof(hostSmall), hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    TCC_REQUIRE(hostSmall[0] == 0, TCC_ERR_INVALID_ARGUMENT, "COO index out of range");

    std::uint32_t* perm = permA;
    std::uint64_t* sorted = keysA;
    if (E > 0) {
        hipLaunchKernelGGL(sw_keys_kernel, dim3(grid_for(E, kBuildThreads)), dim3(kBuildThreads), 0, st, dRow, dCol, E,
                           rowRank, colRank, colBits, keysA, permA);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(radix_sort_pairs(keysA, keysB, permA, permB, E, groupBits + colBits + 6, temp, &sorted, &perm,
                                       st));
        hipLaunchKernelGGL(sw_flags_kernel, dim3(grid_for(E, kBuildThreads)), dim3(kBuildThreads), 0, st, sorted, E,
                           colBits, flags, groupPairs, small);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(flags, pos, E, small + 1, temp, st));
    }
    // Phases: cut points in column-rank order at pair-count quantiles; then
    // units per (phase, super-window), phase first.
    TCC_HIP_CHECK(fill<std::uint32_t>(rankPairs, numCols, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(phaseCounts, GP, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(bounds, kSwMaxPhases, numCols, st));
    if (E > 0) {
        hipLaunchKernelGGL(rank_pairs_kernel, dim3(grid_for(E, kBuildThreads)), dim3(kBuildThreads), 0, st, sorted, flags,
                           E, (1ull << colBits) - 1ull, rankPairs);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(rankPairs, rankCum, numCols, nullptr, temp, st));
        hipLaunchKernelGGL(phase_bounds_kernel, dim3(grid_for(numCols, kBuildThreads)), dim3(kBuildThreads), 0, st,
                           rankCum, numCols, small + 1, phases, bounds);
        hipLaunchKernelGGL(phase_counts_kernel, dim3(grid_for(E, kBuildThreads)), dim3(kBuildThreads), 0, st, sorted,
                           flags, E, colBits, bounds, phases, G, phaseCounts);
        TCC_LAUNCH_CHECK();
    }
    hipLaunchKernelGGL(phase_units_kernel, dim3(grid_for(GP, kBuildThreads)), dim3(kBuildThreads), 0, st, phaseCounts,
                       groupPairs, G, phases, unitPairs, unitCount);
    TCC_LAUNCH_CHECK();
    TCC_HIP_CHECK(exclusive_scan(unitCount, unitCount, GP, small + 2, temp, st));
    TCC_HIP_CHECK(hipMemcpyAsync(hostSmall, small, sizeof(hostSmall), hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    TCC_REQUIRE(hostSmall[0] == 0, TCC_ERR_INVALID_ARGUMENT,
                hostSmall[0] == 2 ? "duplicate (row, col) entries in the COO input" : "COO index out of range");
    const std::uint32_t P = E > 0 ? hostSmall[1] : 0;
    const std::uint32_t U = hostSmall[2];

    // outputs: rowOrder[64G] groupOffset[G+1] units[3U] pairCol[P] pairValue[P] pairMask[P] data[E]
    const std::uint64_t Pn = std::max<std::uint32_t>(P, 1);
    const std::size_t outBytes = align_up(4ull * padded) + align_up(4ull * (G + 1)) + align_up(12ull * U) +
                                 align_up(4 * Pn) + align_up(4 * Pn) + align_up(8 * Pn) + (dVal ? align_up(4 * En) : 0);
    char* o = nullptr;
    TCC_HIP_CHECK(hipMalloc(&o, outBytes));
    char* q = o;
    auto takeOut = [&](std::size_t bytes) {
        char* p = q;
        q += align_up(bytes);
        return p;
    };
    auto* rowOrder = reinterpret_cast<std::uint32_t*>(takeOut(4ull * padded));
    auto* groupOffset = reinterpret_cast<std::uint32_t*>(takeOut(4ull * (G + 1)));
    auto* units = reinterpret_cast<std::uint32_t*>(takeOut(12ull * U));
    auto* pairCol = reinterpret_cast<std::uint32_t*>(takeOut(4 * Pn));
    auto* pairValue = reinterpret_cast<std::uint32_t*>(takeOut(4 * Pn));
    auto* pairMask = reinterpret_cast<std::uint64_t*>(takeOut(8 * Pn));
    float* data = dVal ? reinterpret_cast<float*>(takeOut(4 * En)) : nullptr;
    auto fail = [&](int rc) {
        (void)hipFree(o);
        return rc;
    };
    if (hipMemcpyAsync(rowOrder, rowOrderTmp.p, 4ull * padded, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        exclusive_scan(groupPairs, groupOffset, G, groupOffset + G, temp, st) != hipSuccess ||
        hipMemcpyAsync(unitCount + GP, small + 2, 4, hipMemcpyDeviceToDevice, st) != hipSuccess ||
        fill<std::uint64_t>(pairMask, Pn, 0ull, st) != hipSuccess) {
        set_last_error("HIP error while initialising super-window BCSR arrays");
        return fail(TCC_ERR_HIP);
    }
    if (E > 0) {
        hipLaunchKernelGGL(sw_place_kernel, dim3(grid_for(E, kBuildThreads)), dim3(kBuildThreads), 0, st, sorted, perm,
                           E, flags, pos, dCol, dVal, pairCol, reinterpret_cast<unsigned long long*>(pairMask),
                           pairValue, data);
    }
    hipLaunchKernelGGL(sw_units_kernel, dim3(grid_for(GP, kBuildThreads)), dim3(kBuildThreads), 0, st, groupOffset,
                       phaseCounts, unitCount, G, phases, unitPairs, units);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        set_last_error("HIP error while building the super-window BCSR");
        return fail(TCC_ERR_HIP);
    }
    out->num_rows = numRows;
    out->num_cols = numCols;
    out->nnz = E;
    out->num_groups = G;
    out->num_pairs = P;
    out->num_units = U;
    out->unit_pairs = unitPairs;
    out->num_phases = phases;
    out->rowOrder = rowOrder;
    out->groupOffset = groupOffset;
    out->pairCol = pairCol;
    out->pairMask = pairMask;
    out->pairValue = pairValue;
    out->data = data;
    out->units = units;
    *allocation = o;
    return TCC_OK;
}

int tcc_sw_bcsr_spmm_packed(const tcc_sw_bcsr* A, const void* packedX, float* Y, std::uint32_t featureDim,
                            int accumulate, void* stream) {
    clear_last_error();
    TCC_REQUIRE(sw_ok(A) && packedX && Y && featureDim >= 1, TCC_ERR_INVALID_ARGUMENT,
                "invalid super-window BCSR SpMM arguments");
    TCC_REQUIRE(reinterpret_cast<std::uintptr_t>(packedX) % 16 == 0, TCC_ERR_INVALID_ARGUMENT,
                "packed buffer must be 16-byte aligned");
    const hipStream_t st = as_stream(stream);
    SwArgs a{};
    a.rowOrder = A->rowOrder;
    a.groupOffset = A->groupOffset;
    a.pairCol = A->pairCol;
    a.pairMask = A->pairMask;
    a.pairValue = A->pairValue;
    a.data = A->data;
    a.units = A->units;
    a.packed = static_cast<const unsigned char*>(packedX);
    a.stride = packed_row_stride(featureDim);
    a.Y = Y;
    a.F = featureDim;
    a.numUnits = A->num_units;
    a.numChunks = (featureDim + kPackChunkF - 1) / kPackChunkF;
    a.accumulate = accumulate;
    const std::uint64_t wgs = static_cast<std::uint64_t>(a.numUnits) * a.numChunks;
    TCC_REQUIRE(wgs <= 0x7FFFFFFFull, TCC_ERR_UNSUPPORTED, "super-window SpMM launch too large");
    if (!accumulate) {
        hipLaunchKernelGGL(sw_zero_shared_kernel, dim3(A->num_units), dim3(256), 0, st, a);
        TCC_LAUNCH_CHECK();
    }
    // 32 pairs per stage: 2 x 20 KB of LDS and 114 VGPRs per workgroup, two
    // workgroups per compute unit (16 pairs measured 24.2 against 21.5 ms at
    // the 233k-node, 114M-nnz configuration; 64 pairs fit one workgroup).
    if (a.data) hipLaunchKernelGGL((sw_gather_kernel<32, true>), dim3(static_cast<unsigned>(wgs)), dim3(kSwThreads), 0, st, a);
    else hipLaunchKernelGGL((sw_gather_kernel<32, false>), dim3(static_cast<unsigned>(wgs)), dim3(kSwThreads), 0, st, a);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

}  // extern "C"
