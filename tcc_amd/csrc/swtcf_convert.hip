// COO -> SWTCF conversion on gfx950 (reference: src/swtcf_convert.cu).
//
// Design (deterministic, no hash table, no atomic ranks):
//   1. Each edge becomes a 64-bit element  sw << kb | dst << loBits | lo
//      (sw = super-window = src / 8S, lo = src - 8S * sw, kb = dstBits +
//      loBits), and a stable LSD radix sort puts the elements in
//      (sw, dst, lo) order: the digits of the low kb bits first, then those
//      of sw.  A COO already ordered by (dst, src) -- listed row by row, as
//      CSR gives it -- needs only the sw digits, since a stable partition of
//      that order by sw is the whole sort: the first pass detects such input
//      and the low-digit passes then return at once.
//   2. The elements of one super-window form a segment, cut into tiles of
//      4096 that never straddle two segments.  In a segment, runs of key >> 3
//      are the (window, dst) groups (degree = run length, bitmap = OR of
//      1 << (lo & 7)), runs of key >> loBits are the distinct rows in slot
//      (dst ascending) order, and the groups of a row are its occurrences.
//   3. A count pass takes, per tile, the group heads per (window, degree),
//      the row heads and the repeated rows per occurrence count; one scan
//      over (bin, tile) gives each tile its offsets inside its segment, and
//      the segment totals give each window its degree-bucket bases (degree 8
//      first) and each super-window its repeat-cache bases.
//   4. An emit pass finds the tile's heads again and writes every output in
//      place: a head's rank in its bin is the tile's offset plus the earlier
//      heads of the tile in that bin, which is the canonical (degree desc,
//      dst asc) tile-row order and (occurrence desc, slot asc) cache order.
// Atomics only count (LDS histograms, error flags), so the output is the
// same run to run and equal to the CPU oracle's canonical form.
#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "primitives.hpp"

namespace tcc {

namespace {

constexpr unsigned kThreads = 256;
constexpr unsigned kWaves = kThreads / kWave;  // 4
constexpr unsigned kRounds = 16;
constexpr unsigned kTile = kThreads * kRounds;  // elements per sort tile and per segment tile
constexpr unsigned kSpan = kWave * kRounds;     // consecutive elements of one wave
constexpr unsigned kMaxLowDigit = 9;            // bits per pass over dst/lo
constexpr unsigned kMaxTopDigit = 8;            // bits per pass over sw
constexpr unsigned kMaxBins = 1u << kMaxLowDigit;
constexpr unsigned kMaxS = TCC_SWTCF_MAX_SUPER_WINDOW_SIZE;
constexpr unsigned kCache = TCC_SWTCF_REPEAT_CACHE_SIZE;
// Elements past a tile's end that its heads read: a row has at most 8S
// elements unless a group has more than 8 (which raises the degree error).
constexpr unsigned kLookahead = 8 * kMaxS + 8;
// Counter bins of a segment tile: [0, 8S) group heads by (wi, degree - 1);
// 8S row heads; 8S + occ - 1 repeated rows by occurrence occ in [2, 32];
// 8S + 32 all group heads.
constexpr unsigned kOccBins = kMaxS - 1;
__host__ __device__ inline unsigned num_bins(unsigned S) { return 8 * S + 33; }
constexpr unsigned kOccStride = kMaxS + 1;  // occBase[s * 33 + occ]

inline unsigned ceil_log2(std::uint64_t x) {
    unsigned b = 0;
    while ((1ull << b) < x) ++b;
    return b;
}

// Element packing and the range checks of buildEdgeKeysKernel (:104-144).
struct ElemParams {
    std::uint32_t rows, cols;
    std::uint32_t span;  // 8S sources per super-window
    unsigned loBits, kb;
    unsigned spanShift;  // log2(span) when span is a power of two, else 0
};

struct Digit {
    unsigned shift, bits;
};

struct Plan {
    ElemParams ep;
    unsigned swBits;
    std::vector<Digit> low, top;
};

inline void split_digits(unsigned shift, unsigned bits, unsigned maxBits, std::vector<Digit>& out) {
    const unsigned passes = (bits + maxBits - 1) / maxBits;
    for (unsigned p = 0; p < passes; ++p) {
        const unsigned w = bits / passes + (p < bits % passes ? 1u : 0u);
        out.push_back({shift, w});
        shift += w;
    }
}

inline Plan make_plan(std::uint32_t rows, std::uint32_t cols, std::uint32_t S, std::uint32_t numSuperWindows) {
    Plan p;
    p.ep.rows = rows;
    p.ep.cols = cols;
    p.ep.span = 8 * S;
    p.ep.loBits = std::max(3u, ceil_log2(8ull * S));
    p.ep.spanShift = (1u << p.ep.loBits) == p.ep.span ? p.ep.loBits : 0u;
    const unsigned dstBits = rows ? std::max(1u, ceil_log2(rows)) : 32u;
    p.ep.kb = dstBits + p.ep.loBits;
    p.swBits = std::max(1u, ceil_log2(numSuperWindows));
    split_digits(0, p.ep.kb, kMaxLowDigit, p.low);
    split_digits(p.ep.kb, p.swBits, kMaxTopDigit, p.top);
    return p;
}

inline std::uint64_t sort_tiles(std::uint64_t E) { return std::max<std::uint64_t>(1, (E + kTile - 1) / kTile); }
inline std::uint64_t segment_tiles_max(std::uint64_t E, std::uint64_t SW) { return (E + kTile - 1) / kTile + SW; }

// What a segment tile's workgroup needs first, in one 16-byte load: its
// super-window, first element, the super-window's end and first tile.
struct TileInfo {
    std::uint32_t s, start, segEnd, firstTile;
};

// Byte layout of the workspace scratch allocation.
struct Carve {
    std::uint64_t* elemA;
    std::uint64_t* elemB;
    std::uint32_t* histLow;    // [512 * TM + 1] digit counts, (digit, tile) order, per sort or segment tile
    std::uint32_t* histTop;    // [512 * TM + 1]
    std::uint32_t* counters;   // [bins * TM + 1] segment-tile counts, (bin, tile) order
    std::uint32_t* segStart;   // [SW+1]
    std::uint32_t* firstTile;  // [SW+1]
    TileInfo* tileInfo;        // [TM]
    std::uint32_t* wdBase;     // [CW*8]
    std::uint32_t* wActive;    // [CW]
    std::uint32_t* wTiles;     // [CW]
    std::uint32_t* occBase;    // [SW*33]
    std::uint32_t* flags;      // [4]: [0] = input not in (dst, src) order
    std::uint32_t* temp;       // scan scratch
    std::size_t bytes;
};

inline std::size_t align_up(std::size_t x) { return (x + 255) & ~std::size_t(255); }

inline Carve carve(char* base, std::uint64_t E, std::uint64_t CW, std::uint64_t SW, std::uint32_t S) {
    Carve c{};
    std::size_t off = 0;
    auto take = [&](std::size_t bytes) {
        char* p = base ? base + off : nullptr;
        off = align_up(off + bytes);
        return p;
    };
    // digit counts per sort tile, or (the 32-bit flow's segmented passes)
    // per segment tile, with room for the scan's total
    const std::uint64_t hist = static_cast<std::uint64_t>(kMaxBins) * segment_tiles_max(E, SW) + 1;
    const std::uint64_t cnt = static_cast<std::uint64_t>(num_bins(S)) * segment_tiles_max(E, SW) + 1;
    c.elemA = reinterpret_cast<std::uint64_t*>(take(8 * E));
    c.elemB = reinterpret_cast<std::uint64_t*>(take(8 * E));
    c.histLow = reinterpret_cast<std::uint32_t*>(take(4 * hist));
    c.histTop = reinterpret_cast<std::uint32_t*>(take(4 * hist));
    c.counters = reinterpret_cast<std::uint32_t*>(take(4 * cnt));
    c.segStart = reinterpret_cast<std::uint32_t*>(take(4 * (SW + 1)));
    c.firstTile = reinterpret_cast<std::uint32_t*>(take(4 * (SW + 1)));
    c.tileInfo = reinterpret_cast<TileInfo*>(take(sizeof(TileInfo) * segment_tiles_max(E, SW)));
    c.wdBase = reinterpret_cast<std::uint32_t*>(take(4 * CW * 8));
    c.wActive = reinterpret_cast<std::uint32_t*>(take(4 * CW));
    c.wTiles = reinterpret_cast<std::uint32_t*>(take(4 * CW));
    c.occBase = reinterpret_cast<std::uint32_t*>(take(4 * SW * kOccStride));
    c.flags = reinterpret_cast<std::uint32_t*>(take(4 * 4));
    const std::uint64_t tempElems = std::max({scan_temp_elems(hist), scan_temp_elems(cnt), scan_temp_elems(CW + 1),
                                              scan_temp_elems(SW + 1)});
    c.temp = reinterpret_cast<std::uint32_t*>(take(4 * tempElems));
    c.bytes = off;
    return c;
}

// ---------------------------------------------------------------- sort

__device__ __forceinline__ bool edge_in_range(std::uint32_t d, std::uint32_t s, const ElemParams& p) {
    return s < p.cols && (p.rows == 0 || d < p.rows);
}

// Out-of-range edges become (0, 0), so every later index stays in range; the
// input pass flags the conversion as invalid.
__device__ __forceinline__ std::uint64_t make_elem(std::uint32_t d, std::uint32_t s, const ElemParams& p) {
    if (!edge_in_range(d, s, p)) {
        d = 0;
        s = 0;
    }
    const std::uint32_t sw = p.spanShift ? s >> p.spanShift : s / p.span;
    const std::uint32_t lo = s - sw * p.span;
    return (static_cast<std::uint64_t>(sw) << p.kb) | (static_cast<std::uint64_t>(d) << p.loBits) | lo;
}

__device__ __forceinline__ std::uint64_t clamp_to(std::uint64_t i, std::uint64_t last) { return i < last ? i : last; }

__device__ __forceinline__ unsigned digit_of(std::uint64_t e, Digit d) {
    return static_cast<unsigned>(e >> d.shift) & ((1u << d.bits) - 1u);
}

// Lanes (among `active`) whose nbits-wide key equals this lane's.
__device__ __forceinline__ std::uint64_t match_peers_bits(unsigned key, bool active, unsigned nbits) {
    std::uint64_t peers = __ballot(active);
    for (unsigned b = 0; b < nbits; ++b) {
        const bool bit = (key >> b) & 1u;
        const std::uint64_t m = __ballot(bit);
        peers &= bit ? m : ~m;
    }
    return active ? peers : 0ull;
}

// Reads the COO once: range checks, whether it is in (dst, src) order, and
// the per-tile counts of the first low digit and of the first sw digit (the
// latter is the first pass's histogram when the input is in order).
__global__ void __launch_bounds__(kThreads) input_pass_kernel(const std::uint32_t* __restrict__ dst,
                                                             const std::uint32_t* __restrict__ src, std::uint32_t n,
                                                             ElemParams ep, Digit low, std::uint32_t* __restrict__ histLow,
                                                             Digit top, std::uint32_t* __restrict__ histTop,
                                                             unsigned tiles, std::uint32_t* __restrict__ unsorted,
                                                             std::uint32_t* __restrict__ err) {
    __shared__ std::uint32_t hl[kWaves][kMaxBins];
    __shared__ std::uint32_t ht[kWaves][kMaxBins];
    const unsigned lane = __lane_id();
    const unsigned wave = threadIdx.x / kWave;
    for (unsigned i = threadIdx.x; i < kWaves * kMaxBins; i += kThreads) {
        (&hl[0][0])[i] = 0;
        (&ht[0][0])[i] = 0;
    }
    __syncthreads();
    const std::uint64_t base = static_cast<std::uint64_t>(blockIdx.x) * kTile + wave * kSpan;
    bool outOfOrder = false, srcBad = false, dstBad = false;
    std::uint32_t dv[kRounds], sv[kRounds];
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) {
        const std::uint64_t i = clamp_to(base + r * kWave + lane, n - 1);
        dv[r] = dst[i];
        sv[r] = src[i];
    }
    // the element before the wave's first (itself for element 0)
    const std::uint64_t before = base > 0 ? clamp_to(base - 1, n - 1) : 0;
    const std::uint32_t d0 = dst[before], s0 = src[before];
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) {
        const std::uint64_t i = base + r * kWave + lane;
        const bool valid = i < n;
        const std::uint32_t d = dv[r], s = sv[r];
        std::uint32_t pd = __shfl_up(d, 1, kWave);
        std::uint32_t ps = __shfl_up(s, 1, kWave);
        if (lane == 0) {
            pd = r == 0 ? d0 : static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(dv[r > 0 ? r - 1 : 0]), kWave - 1));
            ps = r == 0 ? s0 : static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(sv[r > 0 ? r - 1 : 0]), kWave - 1));
        }
        if (valid) {
            if (i > 0 && (d < pd || (d == pd && s < ps))) outOfOrder = true;
            srcBad |= s >= ep.cols;
            dstBad |= ep.rows != 0 && d >= ep.rows;
            const std::uint64_t e = make_elem(d, s, ep);
            if (low.bits) atomicAdd(&hl[wave][digit_of(e, low)], 1u);
            atomicAdd(&ht[wave][digit_of(e, top)], 1u);
        }
    }
    __shared__ std::uint32_t waveOut[kWaves];
    const std::uint64_t anyOut = __ballot(outOfOrder);
    if (lane == 0) waveOut[wave] = anyOut != 0;
    if (srcBad) atomicMax(err, static_cast<std::uint32_t>(TCC_DEVERR_SRC_RANGE));
    if (dstBad) atomicMax(err, static_cast<std::uint32_t>(TCC_DEVERR_DST_RANGE));
    __syncthreads();
    // one atomic per workgroup, and none once the flag is seen set (atomics
    // on one address from every wave serialise)
    if (threadIdx.x == 0 && (waveOut[0] | waveOut[1] | waveOut[2] | waveOut[3]) &&
        __hip_atomic_load(unsorted, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u)
        atomicOr(unsorted, 1u);
    for (unsigned b = threadIdx.x; low.bits && b < (1u << low.bits); b += kThreads) {
        std::uint32_t t = 0;
        for (unsigned w = 0; w < kWaves; ++w) t += hl[w][b];
        histLow[static_cast<std::uint64_t>(b) * tiles + blockIdx.x] = t;
    }
    for (unsigned b = threadIdx.x; b < (1u << top.bits); b += kThreads) {
        std::uint32_t t = 0;
        for (unsigned w = 0; w < kWaves; ++w) t += ht[w][b];
        histTop[static_cast<std::uint64_t>(b) * tiles + blockIdx.x] = t;
    }
}

// Per-tile digit counts of an element array (u64 elements, or u32 ones of
// the 32-bit flow).  With onlyUnsorted, returns at once when the input pass
// found the COO in (dst, src) order.
template <typename T>
__global__ void __launch_bounds__(kThreads) elem_hist_kernel(const T* __restrict__ in, std::uint32_t n,
                                                            Digit dg, std::uint32_t* __restrict__ hist,
                                                            unsigned tiles, const std::uint32_t* __restrict__ unsorted,
                                                            int onlyUnsorted) {
    __shared__ std::uint32_t h[kWaves][kMaxBins];
    if (onlyUnsorted && *unsorted == 0u) return;
    const unsigned lane = __lane_id();
    const unsigned wave = threadIdx.x / kWave;
    for (unsigned i = threadIdx.x; i < kWaves * kMaxBins; i += kThreads) (&h[0][0])[i] = 0;
    __syncthreads();
    const std::uint64_t base = static_cast<std::uint64_t>(blockIdx.x) * kTile + wave * kSpan + lane;
    T k[kRounds];
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) k[r] = in[clamp_to(base + r * kWave, n - 1)];
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r)
        if (base + r * kWave < n) atomicAdd(&h[wave][digit_of(static_cast<std::uint64_t>(k[r]), dg)], 1u);
    __syncthreads();
    for (unsigned b = threadIdx.x; b < (1u << dg.bits); b += kThreads) {
        std::uint32_t t = 0;
        for (unsigned w = 0; w < kWaves; ++w) t += h[w][b];
        hist[static_cast<std::uint64_t>(b) * tiles + blockIdx.x] = t;
    }
}

struct ScatterArgs {
    const std::uint64_t* in;
    std::uint64_t* out;
    const std::uint32_t* dst;
    const std::uint32_t* src;
    ElemParams ep;
    std::uint32_t n;
    Digit dg;
    const std::uint32_t* histScan;  // exclusive scan of the (digit, tile) counts
    unsigned tiles;
    const std::uint32_t* unsorted;
    int onlyUnsorted;  // return at once for a COO in (dst, src) order
    // 0: `in`; 1: the COO; 2: the COO if it is in order, else `in`; 3: the
    // u32 elements `in32` of the 32-bit flow's first pass (sw >> w0 << kb |
    // key), sw's low w0 bits being that pass's digit, which its output order
    // gives: the digit run [d0Start[d], d0Start[d + 1]) holding the position
    int source;
    // out32 (else null): u32 output instead of `out`; outMode 1 writes the
    // key (the low kb bits, at most 31), outMode 2 writes sw >> w0 << kb | key
    std::uint32_t* out32;
    int outMode;
    // last pass only (else null): segStart[sw] takes the smallest position
    // of the elements that may start super-window sw (atomicMin; it holds n
    // before the pass)
    std::uint32_t* segStart;
    std::uint64_t keyMask;
    const std::uint32_t* in32;
    const std::uint32_t* d0Scan;  // source 3: the first pass's scanned counts, d0Start[d] = d0Scan[d * tiles]
    unsigned w0;                  // bits of the first pass's digit
};

// The 16 rounds' elements of a lane (element first + 64 r), all loads
// issued before any is used: indices past the end are clamped to the last
// element (those lanes take no part in what follows).
__device__ __forceinline__ void load_elems(const ScatterArgs& a, bool coo, std::uint64_t first,
                                           std::uint64_t (&k)[kRounds], const std::uint32_t* d0s) {
    const std::uint64_t last = a.n - 1;
    if (a.source == 3) {
        std::uint32_t e[kRounds];
#pragma unroll
        for (unsigned r = 0; r < kRounds; ++r) e[r] = a.in32[clamp_to(first + r * kWave, last)];
        const unsigned kb = a.ep.kb;
        const std::uint32_t keyMask = static_cast<std::uint32_t>(a.keyMask);
        const unsigned runs = 1u << a.w0;
        // the digit run holding a position: the last d with d0Start[d] <= i.
        // One search for the wave's first position (the same for every lane),
        // then each round steps forward from the previous round's last lane:
        // positions only grow, and a run spans many tiles.
        const std::uint32_t i0 = static_cast<std::uint32_t>(
            clamp_to(first - __lane_id(), last));  // lane 0's position in round 0
        unsigned lo = 0, hi = runs;
        while (hi - lo > 1) {
            const unsigned mid = (lo + hi) / 2;
            if (d0s[mid] <= i0) lo = mid;
            else hi = mid;
        }
        unsigned d = lo;
#pragma unroll
        for (unsigned r = 0; r < kRounds; ++r) {
            const std::uint32_t i = static_cast<std::uint32_t>(clamp_to(first + r * kWave, last));
            while (d + 1 < runs && d0s[d + 1] <= i) ++d;
            const std::uint64_t sw = (static_cast<std::uint64_t>(e[r] >> kb) << a.w0) | d;
            k[r] = (sw << kb) | (e[r] & keyMask);
            d = static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<int>(d), kWave - 1));
        }
    } else if (coo) {
        std::uint32_t d[kRounds], s[kRounds];
#pragma unroll
        for (unsigned r = 0; r < kRounds; ++r) {
            const std::uint64_t i = clamp_to(first + r * kWave, last);
            d[r] = a.dst[i];
            s[r] = a.src[i];
        }
#pragma unroll
        for (unsigned r = 0; r < kRounds; ++r) k[r] = make_elem(d[r], s[r], a.ep);
    } else {
#pragma unroll
        for (unsigned r = 0; r < kRounds; ++r) k[r] = a.in[clamp_to(first + r * kWave, last)];
    }
}

// Stable scatter of one digit: position = the (digit, tile) offset + the
// same digit's count in earlier waves of the tile + earlier lanes and rounds
// of this wave.  The tile is first ordered by digit in LDS and then written
// out in that order, so that consecutive lanes write consecutive addresses
// of a digit's run (6.18 against 6.47 ms for a shuffled 114M-edge
// conversion with each lane writing its own elements).
//
// S32 (the 32-bit flow's super-window passes, which write u32 output): the
// tile is staged as its u32 output words, each element's digit and, for the
// segment heads of the last pass, the low w0 bits of its super-window (the
// first pass's digit), 6 bytes an element instead of the 8 of the whole
// key, with digits of at most kMaxTopDigit bits: 31 instead of 46 KB of LDS,
// so four workgroups fit a compute unit instead of three.  The super-window
// of a staged element is (digit << w0) | low bits for source 3, and the digit
// itself for a single pass over all of sw's bits (source 1).
template <bool S32>
__global__ void __launch_bounds__(kThreads) elem_scatter_kernel(ScatterArgs a) {
    constexpr unsigned kB = S32 ? (1u << kMaxTopDigit) : kMaxBins;
    __shared__ std::uint32_t cnt[kWaves][kB];
    __shared__ std::uint32_t gbase[kB];   // global start of (digit, this tile)
    __shared__ std::uint32_t tstart[kB];  // start of the digit's run in the tile
    __shared__ std::uint32_t waveSum[kWaves];
    __shared__ __attribute__((aligned(8))) unsigned char stageRaw[S32 ? 6 * kTile : 8 * kTile];
    __shared__ std::uint32_t d0s[(1u << kMaxTopDigit) + 1];
    std::uint64_t* const stage = reinterpret_cast<std::uint64_t*>(stageRaw);        // !S32: the keys
    std::uint32_t* const stageV = reinterpret_cast<std::uint32_t*>(stageRaw);       // S32: output words
    unsigned char* const stageD = stageRaw + 4 * kTile;                             // S32: digits
    unsigned char* const stageLo = stageRaw + 5 * kTile;                            // S32: sw's low w0 bits
    if (a.onlyUnsorted && *a.unsorted == 0u) return;
    const bool coo = a.source == 1 || (a.source == 2 && *a.unsorted == 0u);
    if (a.source == 3) {
        for (unsigned d = threadIdx.x; d < (1u << a.w0); d += kThreads)
            d0s[d] = a.d0Scan[static_cast<std::uint64_t>(d) * a.tiles];
        __syncthreads();
    }
    const unsigned lane = __lane_id();
    const unsigned wave = threadIdx.x / kWave;
    const unsigned bins = 1u << a.dg.bits;
    for (unsigned i = threadIdx.x; i < kWaves * kB; i += kThreads) (&cnt[0][0])[i] = 0;
    __syncthreads();
    const std::uint64_t tile0 = static_cast<std::uint64_t>(blockIdx.x) * kTile;
    const std::uint64_t base = tile0 + wave * kSpan;
    const std::uint64_t lt = lanemask_lt();
    std::uint64_t k[kRounds];
    std::uint32_t rank[kRounds];
    load_elems(a, coo, base + lane, k, d0s);
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) {
        const std::uint64_t i = base + r * kWave + lane;
        const bool valid = i < a.n;
        const unsigned d = digit_of(k[r], a.dg);
        const std::uint64_t peers = match_peers_bits(d, valid, a.dg.bits);
        const std::uint32_t before = cnt[wave][d];
        rank[r] = before + static_cast<std::uint32_t>(__popcll(peers & lt));
        // one lane per digit group publishes the new count; every lane of the
        // wave read cnt[] above before this write is issued
        if (valid && (peers & lt) == 0) cnt[wave][d] = before + static_cast<std::uint32_t>(__popcll(peers));
    }
    __syncthreads();
    {
        // thread j holds digits 2j and 2j + 1: their per-wave offsets within
        // the digit's run, and the runs' starts (an exclusive scan of the
        // digits' tile counts, in digit order)
        std::uint32_t tot[2] = {0, 0};
#pragma unroll
        for (unsigned q = 0; q < 2; ++q) {
            const unsigned d = 2 * threadIdx.x + q;
            if (d < bins) {
                for (unsigned w = 0; w < kWaves; ++w) {
                    const std::uint32_t c = cnt[w][d];
                    cnt[w][d] = tot[q];
                    tot[q] += c;
                }
                gbase[d] = a.histScan[static_cast<std::uint64_t>(d) * a.tiles + blockIdx.x];
            }
        }
        const std::uint32_t pair = tot[0] + tot[1];
        std::uint32_t inc = pair;
#pragma unroll
        for (unsigned o = 1; o < kWave; o <<= 1) {
            const std::uint32_t y = __shfl_up(inc, o, kWave);
            if (lane >= o) inc += y;
        }
        if (lane == kWave - 1) waveSum[wave] = inc;
        __syncthreads();
        std::uint32_t off = inc - pair;
        for (unsigned w = 0; w < wave; ++w) off += waveSum[w];
        if (2 * threadIdx.x < bins) tstart[2 * threadIdx.x] = off;
        if (2 * threadIdx.x + 1 < bins) tstart[2 * threadIdx.x + 1] = off + tot[0];
        __syncthreads();
#pragma unroll
        for (unsigned r = 0; r < kRounds; ++r) {
            const std::uint64_t i = base + r * kWave + lane;
            if (i < a.n) {
                const unsigned d = digit_of(k[r], a.dg);
                const unsigned q = tstart[d] + cnt[wave][d] + rank[r];
                if constexpr (S32) {
                    const std::uint64_t key = k[r];
                    stageV[q] = a.outMode == 1
                                    ? static_cast<std::uint32_t>(key & a.keyMask)
                                    : static_cast<std::uint32_t>(((key >> (a.ep.kb + a.w0)) << a.ep.kb) |
                                                                 (key & a.keyMask));
                    stageD[q] = static_cast<unsigned char>(d);
                    stageLo[q] = static_cast<unsigned char>((key >> a.ep.kb) & ((1u << a.w0) - 1u));
                } else {
                    stage[q] = k[r];
                }
            }
        }
        __syncthreads();
        const std::uint32_t count = static_cast<std::uint32_t>(clamp_to(kTile, a.n - tile0));
        if constexpr (S32) {
            // the element's super-window: (digit << w0) | its low bits after the
            // first pass (source 3), else the digit (one pass over all of sw)
            const auto sw_of = [&](std::uint32_t p) -> std::uint32_t {
                const std::uint32_t d = stageD[p];
                return a.source == 3 ? (d << a.w0) | stageLo[p] : d;
            };
            for (std::uint32_t p = threadIdx.x; p < count; p += kThreads) {
                const unsigned d = stageD[p];
                const std::uint32_t pos = gbase[d] + (p - tstart[d]);
                a.out32[pos] = stageV[p];
                if (a.segStart) {
                    const std::uint32_t sw = sw_of(p);
                    if (p == tstart[d] || sw_of(p - 1) != sw) atomicMin(&a.segStart[sw], pos);
                }
            }
            return;
        }
        for (std::uint32_t p = threadIdx.x; p < count; p += kThreads) {
            const std::uint64_t key = stage[p];
            const unsigned d = digit_of(key, a.dg);
            const std::uint32_t pos = gbase[d] + (p - tstart[d]);
            if (!a.out32) a.out[pos] = key;
            else if (a.outMode == 1) a.out32[pos] = static_cast<std::uint32_t>(key & a.keyMask);
            else
                a.out32[pos] = static_cast<std::uint32_t>(((key >> (a.ep.kb + a.w0)) << a.ep.kb) | (key & a.keyMask));
            if (a.segStart) {
                // a digit's run in the tile is in (sw, key) order, the earlier
                // passes having sorted every lower bit: only its first element
                // and elements whose sw differs from their neighbour's may
                // start a super-window
                const std::uint32_t sw = static_cast<std::uint32_t>(key >> a.ep.kb);
                if (p == tstart[d] || static_cast<std::uint32_t>(stage[p - 1] >> a.ep.kb) != sw)
                    atomicMin(&a.segStart[sw], pos);
            }
        }
    }
}

// ---------------------------------------------------------------- segments

// segStart[s] = min(segStart[s], segStart[s + 1]) from the end, in one
// workgroup: an empty super-window (still n after the last pass) gets the
// next one's start, and segStart[SW] stays n.
__global__ void __launch_bounds__(kThreads) segment_fix_kernel(std::uint32_t* __restrict__ segStart,
                                                               std::uint32_t SW) {
    __shared__ std::uint32_t chunkMin[kThreads];
    const std::uint32_t total = SW + 1;
    const std::uint32_t chunk = (total + kThreads - 1) / kThreads;
    const std::uint32_t b = min(threadIdx.x * chunk, total), e = min(b + chunk, total);
    std::uint32_t m = 0xFFFFFFFFu;
    for (std::uint32_t i = b; i < e; ++i) m = min(m, segStart[i]);
    chunkMin[threadIdx.x] = m;
    __syncthreads();
    std::uint32_t run = 0xFFFFFFFFu;  // min over the later chunks
    for (unsigned t = threadIdx.x + 1; t < kThreads; ++t) run = min(run, chunkMin[t]);
    for (std::uint32_t i = e; i > b; --i) {
        run = min(run, segStart[i - 1]);
        segStart[i - 1] = run;
    }
}

__global__ void segment_tiles_kernel(const std::uint32_t* __restrict__ segStart, std::uint32_t SW,
                                     std::uint32_t* __restrict__ tileCount) {
    const std::uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s < SW) tileCount[s] = (segStart[s + 1] - segStart[s] + kTile - 1) / kTile;
}

__global__ void tile_info_kernel(const std::uint32_t* __restrict__ segStart,
                                 const std::uint32_t* __restrict__ firstTile, std::uint32_t SW,
                                 TileInfo* __restrict__ info) {
    const std::uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s >= SW) return;
    const std::uint32_t t0 = firstTile[s], t1 = firstTile[s + 1], b = segStart[s], e = segStart[s + 1];
    for (std::uint32_t t = t0; t < t1; ++t) info[t] = TileInfo{s, b + (t - t0) * kTile, e, t0};
}

// ---------------------------------------------------------------- segmented passes

// The 32-bit flow partitions by sw first and then, for a COO out of (dst,
// src) order, sorts each super-window's keys: stable LSD passes over u32
// keys whose tiles are the segment tiles, so that a key's position is its
// segment's start + the segment's keys of smaller digits + the same digit's
// keys in the segment's earlier tiles + its rank in the tile.
struct SegPassArgs {
    const std::uint32_t* in;
    std::uint32_t* out;
    const TileInfo* tileInfo;
    const std::uint32_t* firstTile;
    const std::uint32_t* segStart;
    std::uint32_t n, SW, TM;
    Digit dg;
    std::uint32_t* counters;  // [bins][TM] + 1: per-tile digit counts, scanned between the two kernels
    const std::uint32_t* unsorted;
};

// A segment tile's keys, 16 rounds a wave (indices clamped into the tile).
__device__ __forceinline__ void load_seg_keys(const std::uint32_t* __restrict__ in, std::uint32_t start,
                                              std::uint32_t n, unsigned wave, unsigned lane,
                                              std::uint32_t (&k)[kRounds]) {
    const std::uint32_t last = start + (n > 0 ? n - 1 : 0u);
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) k[r] = in[min(start + wave * kSpan + r * kWave + lane, last)];
}

__global__ void __launch_bounds__(kThreads) seg_hist_kernel(SegPassArgs a) {
    __shared__ std::uint32_t h[kWaves][kMaxBins];
    if (*a.unsorted == 0u) return;
    const unsigned t = blockIdx.x, bins = 1u << a.dg.bits;
    const std::uint32_t numTiles = a.firstTile[a.SW];
    const TileInfo ti = a.tileInfo[t];
    if (t >= numTiles) {  // past the last tile: empty columns of the scan
        for (unsigned b = threadIdx.x; b < bins; b += kThreads) a.counters[static_cast<std::uint64_t>(b) * a.TM + t] = 0;
        return;
    }
    const unsigned lane = __lane_id(), wave = threadIdx.x / kWave;
    for (unsigned i = threadIdx.x; i < kWaves * kMaxBins; i += kThreads) (&h[0][0])[i] = 0;
    __syncthreads();
    const std::uint32_t segEnd = min(ti.segEnd, a.n), start = min(ti.start, segEnd);
    const std::uint32_t n = min(kTile, segEnd - start);
    std::uint32_t k[kRounds];
    load_seg_keys(a.in, start, n, wave, lane, k);
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r)
        if (wave * kSpan + r * kWave + lane < n) atomicAdd(&h[wave][digit_of(k[r], a.dg)], 1u);
    __syncthreads();
    for (unsigned b = threadIdx.x; b < bins; b += kThreads) {
        std::uint32_t c = 0;
        for (unsigned w = 0; w < kWaves; ++w) c += h[w][b];
        a.counters[static_cast<std::uint64_t>(b) * a.TM + t] = c;
    }
}

// Exclusive scan over the block of one value per thread (thread order).
__device__ __forceinline__ std::uint32_t block_exclusive_scan(std::uint32_t v, std::uint32_t* waveSum) {
    const unsigned lane = __lane_id(), wave = threadIdx.x / kWave;
    std::uint32_t inc = v;
#pragma unroll
    for (unsigned o = 1; o < kWave; o <<= 1) {
        const std::uint32_t y = __shfl_up(inc, o, kWave);
        if (lane >= o) inc += y;
    }
    if (lane == kWave - 1) waveSum[wave] = inc;
    __syncthreads();
    std::uint32_t off = inc - v;
    for (unsigned w = 0; w < wave; ++w) off += waveSum[w];
    __syncthreads();  // waveSum free for the next scan
    return off;
}

__global__ void __launch_bounds__(kThreads) seg_scatter_kernel(SegPassArgs a) {
    __shared__ std::uint32_t cnt[kWaves][kMaxBins];
    __shared__ std::uint32_t gbase[kMaxBins];   // output position of the digit's first key of this tile
    __shared__ std::uint32_t tstart[kMaxBins];  // start of the digit's run in the staged tile
    __shared__ std::uint32_t waveSum[kWaves];
    __shared__ std::uint32_t stage[kTile];
    if (*a.unsorted == 0u) return;
    const unsigned t = blockIdx.x, bins = 1u << a.dg.bits;
    const std::uint32_t numTiles = a.firstTile[a.SW];
    const TileInfo ti = a.tileInfo[t];
    if (t >= numTiles) return;
    const unsigned lane = __lane_id(), wave = threadIdx.x / kWave;
    const std::uint32_t s = ti.s, t0 = ti.firstTile;
    const std::uint32_t t1 = a.firstTile[s + 1], segBegin = a.segStart[s];
    const std::uint32_t segEnd = min(ti.segEnd, a.n), start = min(ti.start, segEnd);
    const std::uint32_t n = min(kTile, segEnd - start);
    for (unsigned i = threadIdx.x; i < kWaves * kMaxBins; i += kThreads) (&cnt[0][0])[i] = 0;
    __syncthreads();
    std::uint32_t k[kRounds], rank[kRounds];
    load_seg_keys(a.in, start, n, wave, lane, k);
    const std::uint64_t lt = lanemask_lt();
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) {
        const bool valid = wave * kSpan + r * kWave + lane < n;
        const unsigned d = digit_of(k[r], a.dg);
        const std::uint64_t peers = match_peers_bits(d, valid, a.dg.bits);
        const std::uint32_t before = cnt[wave][d];
        rank[r] = before + static_cast<std::uint32_t>(__popcll(peers & lt));
        if (valid && (peers & lt) == 0) cnt[wave][d] = before + static_cast<std::uint32_t>(__popcll(peers));
    }
    __syncthreads();
    // thread j holds digits 2j and 2j + 1: per-wave offsets within the
    // digit's run, the runs' starts in the tile, and the digits' bases in the
    // segment (its keys of smaller digits + this digit's in earlier tiles)
    std::uint32_t tot[2] = {0, 0}, segTot[2] = {0, 0}, earlier[2] = {0, 0};
#pragma unroll
    for (unsigned q = 0; q < 2; ++q) {
        const unsigned d = 2 * threadIdx.x + q;
        if (d < bins) {
            for (unsigned w = 0; w < kWaves; ++w) {
                const std::uint32_t c = cnt[w][d];
                cnt[w][d] = tot[q];
                tot[q] += c;
            }
            const std::uint64_t row = static_cast<std::uint64_t>(d) * a.TM;
            const std::uint32_t p0 = a.counters[row + t0];
            segTot[q] = a.counters[row + t1] - p0;
            earlier[q] = a.counters[row + t] - p0;
        }
    }
    const std::uint32_t ts = block_exclusive_scan(tot[0] + tot[1], waveSum);
    const std::uint32_t sp = block_exclusive_scan(segTot[0] + segTot[1], waveSum);
    if (2 * threadIdx.x < bins) {
        tstart[2 * threadIdx.x] = ts;
        gbase[2 * threadIdx.x] = segBegin + sp + earlier[0];
    }
    if (2 * threadIdx.x + 1 < bins) {
        tstart[2 * threadIdx.x + 1] = ts + tot[0];
        gbase[2 * threadIdx.x + 1] = segBegin + sp + segTot[0] + earlier[1];
    }
    __syncthreads();
#pragma unroll
    for (unsigned r = 0; r < kRounds; ++r) {
        if (wave * kSpan + r * kWave + lane < n) {
            const unsigned d = digit_of(k[r], a.dg);
            stage[tstart[d] + cnt[wave][d] + rank[r]] = k[r];
        }
    }
    __syncthreads();
    for (std::uint32_t p = threadIdx.x; p < n; p += kThreads) {
        const std::uint32_t key = stage[p];
        const unsigned d = digit_of(key, a.dg);
        a.out[gbase[d] + (p - tstart[d])] = key;
    }
}

struct TileArgs {
    const std::uint64_t* el;      // the sorted elements (keys of more than 31 bits)
    const std::uint32_t* keys32;  // or their low kb bits
    // the 32-bit flow: the keys are in keys32Unsorted when the segmented
    // passes ran (a COO out of order, *unsorted set), else in keys32; the
    // head facts then follow them in the same buffer (null: keys32 and info)
    const std::uint32_t* keys32Unsorted;
    const std::uint32_t* unsorted;
    std::uint32_t n;    // elements
    std::uint32_t cap;  // the matrix's edge capacity (bounds of the row and tile-row arrays)
    std::uint64_t keyMask;  // the low kb bits: dst << loBits | lo
    unsigned loBits;
    std::uint32_t S, SW, CW;
    const std::uint32_t* segStart;
    const std::uint32_t* firstTile;  // [SW+1] exclusive scan of tiles per segment
    const TileInfo* tileInfo;        // [tiles]
    std::uint32_t* counters;         // [bins][TM] (+1), scanned before the emit pass
    std::uint32_t* info;             // [n] head facts of each element (count pass -> emit pass)

    __device__ const std::uint32_t* keys() const {
        return unsorted && *unsorted ? keys32Unsorted : keys32;
    }
    __device__ std::uint32_t* facts() const {
        return unsorted ? const_cast<std::uint32_t*>(keys()) + n : info;
    }
    std::uint32_t TM;
    std::uint32_t* err;
    // emit pass
    const std::uint32_t* wdBase;
    const std::uint32_t* colWindowOffset;
    const std::uint32_t* occBase;
    std::uint32_t* tileRowSlot;
    std::uint8_t* tileBytes;
    std::uint32_t* superWindowRows;
    std::uint8_t* rowCacheSlot;
    std::uint32_t* cachedRowSlot;
};

struct TileRange {
    std::uint32_t s, t0, start, n, avail;
};

constexpr unsigned kKeySlots = 1 + kTile + kLookahead;
constexpr unsigned kFlagWords = (kTile + kLookahead + kWave - 1) / kWave;
// The emit pass runs 8 waves on a tile (8 rounds of 64 each): half the
// per-lane rank registers of 4 waves, so twice the waves per SIMD.
constexpr unsigned kEmitThreads = 512;
constexpr unsigned kEmitWaves = kEmitThreads / kWave;
constexpr unsigned kEmitRounds = kTile / kEmitThreads;
constexpr unsigned kEmitSpan = kWave * kEmitRounds;

// The keys of a segment tile and its head bitmaps.  K is u32 when the keys
// have at most 31 bits (so that the ~0 sentinel never equals a key shifted
// right), else u64.
template <typename K>
struct TileKeys {
    K key[kKeySlots];                 // key[0]: element before the tile, or ~0; key[1 + i]: element i
    // bit i: element i starts a (window, dst) group / a row; two spare words
    // so that 64-bit windows may read past the last one written (those bits
    // lie at or past avail and are masked)
    std::uint64_t group[kFlagWords + 2];
    std::uint64_t row[kFlagWords + 2];
};

// Segment tile t: its elements, up to kLookahead elements past its end
// (within the super-window), and the head bits of all of them.
template <unsigned THREADS, typename K>
__device__ TileRange load_tile(const TileArgs& a, unsigned t, const TileInfo& ti, TileKeys<K>& tk) {
    constexpr unsigned kLoadIters = (kKeySlots + THREADS - 1) / THREADS;
    TileRange r;
    r.s = ti.s;
    r.t0 = ti.firstTile;
    const std::uint32_t segEnd = min(ti.segEnd, a.n);
    r.start = min(ti.start, segEnd);
    r.n = min(kTile, segEnd - r.start);
    r.avail = min(r.n + kLookahead, segEnd - r.start);
    const bool hasPrev = t > ti.firstTile;
    // all loads issued before any is stored: indices clamped into the
    // segment, the slot before a segment's first element set to ~0 after
    std::uint64_t v[kLoadIters];
    const std::uint32_t first = hasPrev ? r.start - 1 : r.start;
    const std::uint32_t* keys32 = a.keys();
#pragma unroll
    for (unsigned q = 0; q < kLoadIters; ++q) {
        const unsigned j = q * THREADS + threadIdx.x;
        const std::uint32_t e = min(first + j, segEnd > 0 ? segEnd - 1 : 0u);
        if constexpr (sizeof(K) == 4) v[q] = keys32[e];
        else v[q] = a.el[e];
    }
#pragma unroll
    for (unsigned q = 0; q < kLoadIters; ++q) {
        const unsigned j = q * THREADS + threadIdx.x;
        // key[j] = element start - 1 + j
        if (hasPrev) {
            if (j <= r.avail) tk.key[j] = static_cast<K>(v[q] & a.keyMask);
        } else if (j < r.avail) {
            tk.key[j + 1] = static_cast<K>(v[q] & a.keyMask);
        }
    }
    if (!hasPrev && threadIdx.x == 0) tk.key[0] = static_cast<K>(~0ull);
    __syncthreads();
    const unsigned lane = __lane_id();
    for (unsigned base = (threadIdx.x / kWave) * kWave; base < r.avail; base += THREADS) {
        const unsigned j = base + lane;
        bool g = false, h = false;
        if (j < r.avail) {
            const K x = tk.key[j + 1], p = tk.key[j];
            g = (x >> 3) != (p >> 3);
            h = (x >> a.loBits) != (p >> a.loBits);
        }
        const std::uint64_t gb = __ballot(g), rb = __ballot(h);
        if (lane == 0) {
            tk.group[base / kWave] = gb;
            tk.row[base / kWave] = rb;
        }
    }
    __syncthreads();
    return r;
}

__device__ __forceinline__ bool bit_at(const std::uint64_t* w, unsigned i) { return (w[i >> 6] >> (i & 63)) & 1ull; }

// First set bit in [from, limit), or limit.
__device__ __forceinline__ unsigned next_bit(const std::uint64_t* w, unsigned from, unsigned limit) {
    if (from >= limit) return limit;
    unsigned k = from >> 6;
    std::uint64_t m = w[k] & (~0ull << (from & 63));
    while (m == 0) {
        ++k;
        if (k * 64 >= limit) return limit;
        m = w[k];
    }
    return min(k * 64 + static_cast<unsigned>(__builtin_ctzll(m)), limit);
}

// Set bits in [from, to).
__device__ __forceinline__ unsigned count_bits(const std::uint64_t* w, unsigned from, unsigned to) {
    unsigned c = 0;
    for (unsigned k = from >> 6; k * 64 < to; ++k) {
        std::uint64_t m = w[k];
        if (k == (from >> 6)) m &= ~0ull << (from & 63);
        if (to - k * 64 < 64) m &= (1ull << (to - k * 64)) - 1ull;
        c += static_cast<unsigned>(__popcll(m));
    }
    return c;
}

// Head facts of an element, one u32 written by the count pass for the emit
// pass: group head | row head << 1 | repeated row << 2 | degree << 3 |
// group bitmap << 7 | wi << 15 | (occurrences - 2) << 20.
constexpr std::uint32_t kInfoGroup = 1u, kInfoRow = 2u, kInfoRepeat = 4u;

struct Head {
    bool gh, rh;     // first element of its (window, dst) group / of its row
    unsigned count;  // group: elements, up to 9 (more than 8 is the degree error)
    unsigned bits;   // group: OR of 1 << (lo & 7) over its first 8 elements
    unsigned occ;    // row: groups in the row
};

// Bits [i, i + 64) of a bitmap.
__device__ __forceinline__ std::uint64_t window64(const std::uint64_t* w, unsigned i) {
    const unsigned k = i >> 6, sh = i & 63;
    const std::uint64_t lo = w[k], hi = w[k + 1];
    return sh ? (lo >> sh) | (hi << (64 - sh)) : lo;
}

// Element i of the tile; elements [0, avail) are loaded.  A group ends at
// the next group head (a row head is one too), a row at the next row head:
// both found in a 64-bit window of the head bits (groups have at most 9
// elements here; rows longer than 64 take the word loop).
template <typename K>
__device__ __forceinline__ Head head_at(const TileKeys<K>& tk, unsigned i, unsigned avail) {
    Head h{};
    h.gh = bit_at(tk.group, i);
    h.rh = bit_at(tk.row, i);
    if (h.gh) {
        const std::uint64_t after = window64(tk.group, i + 1) | (1ull << 8);
        h.count = min(static_cast<unsigned>(__builtin_ctzll(after)) + 1, avail - i);
        const unsigned deg = min(h.count, 8u);
        // eight unconditional reads (slots past the loaded elements are in
        // the array and masked), so they issue together
        unsigned bits = 0;
#pragma unroll
        for (unsigned q = 0; q < 8; ++q) {
            const unsigned b = 1u << static_cast<unsigned>(tk.key[i + 1 + q] & 7u);
            bits |= q < deg ? b : 0u;
        }
        h.bits = bits;
    }
    if (h.rh) {
        const std::uint64_t after = window64(tk.row, i + 1);
        if (after != 0 && static_cast<unsigned>(__builtin_ctzll(after)) + 1 <= avail - i) {
            const unsigned len = static_cast<unsigned>(__builtin_ctzll(after)) + 1;  // <= 64
            const std::uint64_t mask = len == 64 ? ~0ull : (1ull << len) - 1ull;
            h.occ = static_cast<unsigned>(__popcll(window64(tk.group, i) & mask));
        } else {
            h.occ = count_bits(tk.group, i, next_bit(tk.row, i + 1, avail));
        }
    }
    return h;
}

// countWindowDegreesKernel (:147-213) and the occurrence counts of
// buildRepeatCacheMetadataKernel (:699-895), per segment tile.
template <typename K>
__global__ void __launch_bounds__(kThreads) tile_count_kernel(TileArgs a) {
    __shared__ TileKeys<K> tk;
    __shared__ std::uint32_t hist[8 * kMaxS + 33];
    const unsigned t = blockIdx.x;
    const unsigned nb = num_bins(a.S);
    // both loads before the branch (tileInfo past the last tile is unused)
    const std::uint32_t numTiles = a.firstTile[a.SW];
    const TileInfo ti = a.tileInfo[t];
    if (t >= numTiles) {  // past the last tile: empty columns of the scan
        for (unsigned b = threadIdx.x; b < nb; b += kThreads) a.counters[static_cast<std::uint64_t>(b) * a.TM + t] = 0;
        return;
    }
    for (unsigned b = threadIdx.x; b < nb; b += kThreads) hist[b] = 0;
    const TileRange r = load_tile<kThreads>(a, t, ti, tk);
    std::uint32_t* facts = a.facts();
    const std::uint32_t loMask = (1u << a.loBits) - 1u;
    const unsigned rowBin = 8 * a.S, groupBin = 8 * a.S + 32;
    std::uint32_t groups = 0, rows = 0;
    bool degErr = false, occErr = false;
    for (unsigned i = threadIdx.x; i < r.n; i += kThreads) {
        const Head h = head_at(tk, i, r.avail);
        const unsigned deg = h.gh ? min(h.count, 8u) : 1u;
        const unsigned wi = (static_cast<std::uint32_t>(tk.key[i + 1]) & loMask) >> 3;
        const bool rep = h.rh && h.occ >= 2 && h.occ <= kMaxS;
        if (h.gh) {
            degErr |= h.count > 8;
            atomicAdd(&hist[wi * 8 + deg - 1], 1u);
            ++groups;
        }
        if (h.rh) {
            ++rows;
            occErr |= h.occ > kMaxS;
            if (rep) atomicAdd(&hist[rowBin + h.occ - 1], 1u);
        }
        facts[r.start + i] = (h.gh ? kInfoGroup : 0u) | (h.rh ? kInfoRow : 0u) | (rep ? kInfoRepeat : 0u) |
                              (deg << 3) | ((h.gh ? h.bits : 0u) << 7) | (min(wi, 31u) << 15) |
                              ((rep ? h.occ - 2 : 0u) << 20);
    }
    if (degErr) atomicMax(a.err, static_cast<std::uint32_t>(TCC_DEVERR_DEGREE));
    if (occErr) atomicMax(a.err, static_cast<std::uint32_t>(TCC_DEVERR_OCCURRENCE));
    if (groups) atomicAdd(&hist[groupBin], groups);
    if (rows) atomicAdd(&hist[rowBin], rows);
    __syncthreads();
    for (unsigned b = threadIdx.x; b < nb; b += kThreads) a.counters[static_cast<std::uint64_t>(b) * a.TM + t] = hist[b];
}

// buildWindowMetadataKernel (:216-265): per window, the degree-bucket bases
// (degree 8 first) from its super-window's totals.
__global__ void window_meta_kernel(const std::uint32_t* __restrict__ P, std::uint32_t TM,
                                   const std::uint32_t* __restrict__ firstTile, std::uint32_t S, std::uint32_t CW,
                                   std::uint32_t* __restrict__ wdBase, std::uint32_t* __restrict__ wActive,
                                   std::uint32_t* __restrict__ wTiles) {
    const std::uint32_t w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= CW) return;
    const std::uint32_t s = w / S, wi = w - s * S;
    const std::uint32_t t0 = firstTile[s], t1 = firstTile[s + 1];
    std::uint32_t running = 0;
    for (int d = 7; d >= 0; --d) {
        const std::uint64_t b = static_cast<std::uint64_t>(wi * 8 + d) * TM;
        wdBase[static_cast<std::uint64_t>(w) * 8 + d] = running;
        running += P[b + t1] - P[b + t0];
    }
    wActive[w] = running;
    wTiles[w] = (running + 7) / 8;
}

// Per super-window: superWindowRowOffset, the repeat-cache bases
// (occurrence 32 first) and the cached count; thread SW writes the totals.
__global__ void super_window_meta_kernel(const std::uint32_t* __restrict__ P, std::uint32_t TM,
                                         const std::uint32_t* __restrict__ firstTile, std::uint32_t S,
                                         std::uint32_t SW, std::uint32_t* __restrict__ occBase,
                                         std::uint32_t* __restrict__ superWindowRowOffset,
                                         std::uint8_t* __restrict__ cachedCount,
                                         std::uint32_t* __restrict__ numGroups) {
    const std::uint32_t s = blockIdx.x * blockDim.x + threadIdx.x;
    if (s > SW) return;
    const std::uint64_t rowBin = static_cast<std::uint64_t>(8 * S) * TM;
    superWindowRowOffset[s] = P[rowBin + firstTile[s]] - P[rowBin];
    if (s == SW) {
        const std::uint64_t groupBin = static_cast<std::uint64_t>(8 * S + 32) * TM;
        *numGroups = P[groupBin + TM] - P[groupBin];
        return;
    }
    const std::uint32_t t0 = firstTile[s], t1 = firstTile[s + 1];
    std::uint32_t running = 0;
    for (unsigned occ = kMaxS; occ >= 2; --occ) {
        const std::uint64_t b = static_cast<std::uint64_t>(8 * S + occ - 1) * TM;
        occBase[static_cast<std::uint64_t>(s) * kOccStride + occ] = running;
        running += P[b + t1] - P[b + t0];
    }
    cachedCount[s] = static_cast<std::uint8_t>(running < kCache ? running : kCache);
}

// assignGroupLocationsKernel (:292-376), fillValidTileRowSlotsKernel
// (:1003-1048), the tile bitmaps (:430-455, one byte per tile row), the
// super-window rows (:459-681) and the repeat cache (:699-895), per segment
// tile, from the head facts of the count pass.  Wave w ranks elements
// [512 w, 512 w + 512) of the tile in 8 rounds of 64, so ranks follow
// element order.
template <typename K>
__global__ void __launch_bounds__(kEmitThreads) tile_emit_kernel(TileArgs a) {
    __shared__ std::uint32_t cntG[kEmitWaves][8 * kMaxS];
    __shared__ std::uint32_t cntO[kEmitWaves][kOccBins + 1];
    __shared__ std::uint64_t baseG[8 * kMaxS];   // tile-row index of the bin's first head in this tile
    __shared__ std::uint32_t baseO[kOccBins + 1];  // cache slot of the bin's first repeated row in this tile
    __shared__ std::uint32_t rowsW[kEmitWaves];
    const unsigned t = blockIdx.x;
    const std::uint32_t numTiles = a.firstTile[a.SW];
    const TileInfo ti = a.tileInfo[t];
    if (t >= numTiles) return;
    const std::uint32_t s = ti.s, t0 = ti.firstTile;
    const std::uint32_t segEnd = min(ti.segEnd, a.n);
    const std::uint32_t start = min(ti.start, segEnd);
    const std::uint32_t n = min(kTile, segEnd - start);
    const unsigned lane = __lane_id();
    const unsigned wave = threadIdx.x / kWave;
    // the wave's head facts and keys, loaded first
    std::uint32_t f[kEmitRounds];
    K key[kEmitRounds];
    const std::uint32_t* keys32 = a.keys();
    const std::uint32_t* facts = a.facts();
#pragma unroll
    for (unsigned r0 = 0; r0 < kEmitRounds; ++r0) {
        const unsigned i = wave * kEmitSpan + r0 * kWave + lane;
        const std::uint32_t e = start + min(i, n - 1);
        f[r0] = facts[e];
        if constexpr (sizeof(K) == 4) key[r0] = keys32[e];
        else key[r0] = a.el[e] & a.keyMask;
        if (i >= n) f[r0] = 0;
    }
    const unsigned groupBins = 8 * a.S;
    for (unsigned b = threadIdx.x; b < groupBins; b += kEmitThreads) {
        // bin b = (wi, degree - 1): the window's degree-bucket base, plus the
        // bucket's heads in the segment's earlier tiles
        const std::uint64_t o = static_cast<std::uint64_t>(b) * a.TM;
        const std::uint32_t w = s * a.S + b / 8;
        const std::uint32_t rel = a.counters[o + t] - a.counters[o + t0];
        baseG[b] = w < a.CW ? static_cast<std::uint64_t>(a.colWindowOffset[w]) * 8 +
                                  a.wdBase[static_cast<std::uint64_t>(w) * 8 + b % 8] + rel
                            : 0;
        for (unsigned v = 0; v < kEmitWaves; ++v) cntG[v][b] = 0;
    }
    for (unsigned b = threadIdx.x; b < kOccBins; b += kEmitThreads) {
        const std::uint64_t o = static_cast<std::uint64_t>(groupBins + 1 + b) * a.TM;
        baseO[b] = a.occBase[static_cast<std::uint64_t>(s) * kOccStride + b + 2] + a.counters[o + t] -
                   a.counters[o + t0];
        for (unsigned v = 0; v < kEmitWaves; ++v) cntO[v][b] = 0;
    }
    const std::uint64_t rowBin = static_cast<std::uint64_t>(groupBins) * a.TM;
    const std::uint32_t rowBase = a.counters[rowBin + t] - a.counters[rowBin];
    const std::uint32_t off0 = a.counters[rowBin + t0] - a.counters[rowBin];
    __syncthreads();

    const std::uint64_t lt = lanemask_lt();
    // ranks per round: group rank | occurrence rank << 10 | rows of the wave
    // up to and including the element << 20 (ranks within the wave)
    std::uint32_t ranks[kEmitRounds];
    std::uint32_t rowRun = 0;
#pragma unroll
    for (unsigned r0 = 0; r0 < kEmitRounds; ++r0) {
        const std::uint32_t fr = f[r0];
        const bool gh = fr & kInfoGroup, rh = fr & kInfoRow, rep = fr & kInfoRepeat;
        const unsigned gbin = gh ? ((fr >> 15) & 31u) * 8 + ((fr >> 3) & 15u) - 1 : 0u;
        const std::uint64_t pg = match_peers<8>(gbin, gh);
        const std::uint32_t bg = cntG[wave][gbin];
        const std::uint32_t rg = bg + static_cast<std::uint32_t>(__popcll(pg & lt));
        if (gh && (pg & lt) == 0) cntG[wave][gbin] = bg + static_cast<std::uint32_t>(__popcll(pg));
        std::uint32_t ro = 0;
        if (__ballot(rep)) {  // repeated rows are rare: most rounds skip this
            const unsigned obin = (fr >> 20) & 31u;
            const std::uint64_t po = match_peers<5>(obin, rep);
            const std::uint32_t bo = cntO[wave][obin];
            ro = bo + static_cast<std::uint32_t>(__popcll(po & lt));
            if (rep && (po & lt) == 0) cntO[wave][obin] = bo + static_cast<std::uint32_t>(__popcll(po));
        }
        const std::uint64_t rb = __ballot(rh);
        const std::uint32_t rowsAt = rowRun + static_cast<std::uint32_t>(__popcll(rb & lt)) + (rh ? 1u : 0u);
        rowRun += static_cast<std::uint32_t>(__popcll(rb));
        ranks[r0] = rg | (ro << 10) | (rowsAt << 20);
    }
    if (lane == 0) rowsW[wave] = rowRun;
    __syncthreads();
    for (unsigned b = threadIdx.x; b < groupBins; b += kEmitThreads) {
        std::uint32_t run = 0;
        for (unsigned w = 0; w < kEmitWaves; ++w) {
            const std::uint32_t c = cntG[w][b];
            cntG[w][b] = run;
            run += c;
        }
    }
    for (unsigned b = threadIdx.x; b < kOccBins; b += kEmitThreads) {
        std::uint32_t run = 0;
        for (unsigned w = 0; w < kEmitWaves; ++w) {
            const std::uint32_t c = cntO[w][b];
            cntO[w][b] = run;
            run += c;
        }
    }
    __syncthreads();
    std::uint32_t rowOff = rowBase;
    for (unsigned w = 0; w < wave; ++w) rowOff += rowsW[w];
#pragma unroll
    for (unsigned r0 = 0; r0 < kEmitRounds; ++r0) {
        const std::uint32_t fr = f[r0];
        if ((fr & (kInfoGroup | kInfoRow)) == 0) continue;
        const std::uint32_t u = rowOff + (ranks[r0] >> 20) - 1;  // this element's row
        const std::uint32_t slot = u - off0;
        const unsigned wi = (fr >> 15) & 31u;
        if ((fr & kInfoGroup) && wi < a.S) {
            // tiles of a window are consecutive: tile-row index = 8 x the
            // window's first tile + the rank among its groups
            const unsigned gbin = wi * 8 + ((fr >> 3) & 15u) - 1;
            const std::uint64_t loc = baseG[gbin] + cntG[wave][gbin] + (ranks[r0] & 0x3FFu);
            if (loc < 8ull * a.cap) {
                a.tileRowSlot[loc] = slot;
                a.tileBytes[loc] = static_cast<std::uint8_t>((fr >> 7) & 0xFFu);
            }
        }
        if ((fr & kInfoRow) && u < a.cap) {
            a.superWindowRows[u] = static_cast<std::uint32_t>(key[r0] >> a.loBits);
            std::uint8_t cs8 = static_cast<std::uint8_t>(TCC_SWTCF_INVALID_CACHE_SLOT);
            if (fr & kInfoRepeat) {
                const unsigned obin = (fr >> 20) & 31u;
                const std::uint32_t cs = baseO[obin] + cntO[wave][obin] + ((ranks[r0] >> 10) & 0x3FFu);
                if (cs < kCache) {
                    cs8 = static_cast<std::uint8_t>(cs);
                    a.cachedRowSlot[static_cast<std::uint64_t>(s) * kCache + cs] = slot;
                }
            }
            a.rowCacheSlot[u] = cs8;
        }
    }
}

// fillPaddingTileRowSlotsKernel (:1051-1107), and zero bitmap bytes for the
// padding rows of each window's last tile.
__global__ void padding_kernel(const std::uint32_t* __restrict__ wActive,
                               const std::uint32_t* __restrict__ colWindowOffset, std::uint32_t CW,
                               std::uint32_t* __restrict__ tileRowSlot, std::uint8_t* __restrict__ tileBytes) {
    const std::uint32_t w = blockIdx.x * blockDim.x + threadIdx.x;
    if (w >= CW) return;
    const std::uint32_t active = wActive[w];
    const std::uint32_t rem = active & 7u;
    if (active == 0 || rem == 0) return;
    const std::uint64_t last = colWindowOffset[w + 1] - 1;
    for (std::uint32_t lr = rem; lr < 8; ++lr) {
        tileRowSlot[last * 8 + lr] = TCC_SWTCF_INVALID_ROW_SLOT;
        tileBytes[last * 8 + lr] = 0;
    }
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
    const Carve c = carve(nullptr, edgeCapacity, ws->numColWindows, ws->numSuperWindows, superWindowSize);
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
    const Plan plan = make_plan(m->rows, m->cols, S, SW);
    TCC_REQUIRE(plan.ep.kb + plan.swBits <= 64, TCC_ERR_UNSUPPORTED, "packed sort key exceeds 64 bits");
    const Carve c = carve(static_cast<char*>(ws->scratch), ws->edgeCapacity, ws->numColWindows,
                          ws->numSuperWindows, S);
    std::uint32_t* err = ws->deviceError;
    std::uint32_t* unsorted = c.flags;
    const unsigned tiles = static_cast<unsigned>(sort_tiles(E));

    // Per-conversion state (:1789-1919), with fill kernels.  Every row of
    // every tile up to colWindowOffset[CW], and every super-window row, is
    // written below; the rest of the arrays is left as it was.
    TCC_HIP_CHECK(fill<std::uint32_t>(m->superWindowCachedRowSlot, static_cast<std::uint64_t>(SW) * kCache,
                                      TCC_SWTCF_INVALID_ROW_SLOT, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(err, 1, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(unsorted, 1, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(c.segStart, static_cast<std::uint64_t>(SW) + 1, E, st));

    // 1. sort.  The 32-bit flow (keys of at most 31 bits, and the first sw
    // pass's output sw >> w0 << kb | key within 32 bits): the sw digits
    // first, from the COO, then -- only for a COO out of (dst, src) order --
    // the low digits per super-window (step 2).  Otherwise 64-bit elements:
    // the low digits (skipped for a COO in order), then the sw digits.
    const bool narrow = plan.ep.kb <= 31;  // keys fit u32 with room for the ~0 sentinel
    const unsigned w0 = plan.top[0].bits;
    const bool flow32 = narrow && (plan.top.size() == 1 ||
                                   (plan.top.size() == 2 && plan.swBits - w0 + plan.ep.kb <= 32));
    hipLaunchKernelGGL(input_pass_kernel, dim3(tiles), dim3(kThreads), 0, st, dDst, dSrc, E, plan.ep,
                       flow32 ? Digit{0, 0} : plan.low[0], c.histLow, plan.top[0], c.histTop, tiles, unsorted, err);
    TCC_LAUNCH_CHECK();
    std::uint64_t* bufs[2] = {c.elemA, c.elemB};
    std::uint32_t* A32 = reinterpret_cast<std::uint32_t*>(c.elemA);
    std::uint32_t* B32 = reinterpret_cast<std::uint32_t*>(c.elemB);
    const std::uint64_t keyMask = (1ull << plan.ep.kb) - 1ull;
    int next = 0;
    const std::uint64_t* cur = nullptr;
    auto scatter = [&](const Digit& dg, std::uint32_t* hist, int onlyUnsorted, int source, bool last) -> int {
        TCC_HIP_CHECK(exclusive_scan(hist, hist, (1ull << dg.bits) * tiles, nullptr, c.temp, st,
                                     onlyUnsorted ? unsorted : nullptr));
        ScatterArgs a{cur, bufs[next], dDst, dSrc, plan.ep, E, dg, hist, tiles, unsorted, onlyUnsorted, source,
                      last && narrow ? reinterpret_cast<std::uint32_t*>(bufs[next]) : nullptr, 1,
                      last ? c.segStart : nullptr, keyMask, nullptr, nullptr, w0};
        hipLaunchKernelGGL(elem_scatter_kernel<false>, dim3(tiles), dim3(kThreads), 0, st, a);
        TCC_LAUNCH_CHECK();
        cur = bufs[next];
        next ^= 1;
        return TCC_OK;
    };
    if (flow32) {
        // sw pass 0 from the COO (counts from the input pass): the keys and
        // segment heads if it is the only one, else sw >> w0 << kb | key
        const bool one = plan.top.size() == 1;
        TCC_HIP_CHECK(exclusive_scan(c.histTop, c.histTop, (1ull << w0) * tiles, nullptr, c.temp, st));
        ScatterArgs a0{nullptr, nullptr, dDst, dSrc, plan.ep, E, plan.top[0], c.histTop, tiles, unsorted, 0, 1,
                       one ? B32 : A32, one ? 1 : 2, one ? c.segStart : nullptr, keyMask, nullptr, nullptr, w0};
        hipLaunchKernelGGL(elem_scatter_kernel<true>, dim3(tiles), dim3(kThreads), 0, st, a0);
        TCC_LAUNCH_CHECK();
        if (!one) {
            // sw pass 1: sw's low w0 bits from the position in pass 0's output
            const Digit d1{plan.ep.kb, plan.top[1].bits};  // sw >> w0 in the u32 elements
            hipLaunchKernelGGL(elem_hist_kernel<std::uint32_t>, dim3(tiles), dim3(kThreads), 0, st, A32, E, d1,
                               c.histLow, tiles, unsorted, 0);
            TCC_LAUNCH_CHECK();
            TCC_HIP_CHECK(exclusive_scan(c.histLow, c.histLow, (1ull << d1.bits) * tiles, nullptr, c.temp, st));
            ScatterArgs a1{nullptr, nullptr, dDst, dSrc, plan.ep, E, plan.top[1], c.histLow, tiles, unsorted, 0, 3,
                           B32, 1, c.segStart, keyMask, A32, c.histTop, w0};
            hipLaunchKernelGGL(elem_scatter_kernel<true>, dim3(tiles), dim3(kThreads), 0, st, a1);
            TCC_LAUNCH_CHECK();
        }
    } else {
        for (std::size_t p = 0; p < plan.low.size(); ++p) {
            if (p > 0) {
                hipLaunchKernelGGL(elem_hist_kernel<std::uint64_t>, dim3(tiles), dim3(kThreads), 0, st, cur, E,
                                   plan.low[p], c.histLow, tiles, unsorted, 1);
                TCC_LAUNCH_CHECK();
            }
            if (int rc = scatter(plan.low[p], c.histLow, 1, p == 0 ? 1 : 0, false)) return rc;
        }
        for (std::size_t p = 0; p < plan.top.size(); ++p) {
            // pass 0's counts came from the input pass for a COO in order
            hipLaunchKernelGGL(elem_hist_kernel<std::uint64_t>, dim3(tiles), dim3(kThreads), 0, st, cur, E,
                               plan.top[p], c.histTop, tiles, unsorted, p == 0 ? 1 : 0);
            TCC_LAUNCH_CHECK();
            if (int rc = scatter(plan.top[p], c.histTop, 0, p == 0 ? 2 : 0, p + 1 == plan.top.size())) return rc;
        }
    }
    const std::uint64_t* sorted = flow32 ? c.elemB : cur;  // u32 keys when narrow

    // 2. segments (super-windows) and their tiles
    hipLaunchKernelGGL(segment_fix_kernel, dim3(1), dim3(kThreads), 0, st, c.segStart, SW);
    TCC_LAUNCH_CHECK();
    hipLaunchKernelGGL(segment_tiles_kernel, dim3(grid_for(SW, kThreads)), dim3(kThreads), 0, st, c.segStart, SW,
                       c.firstTile);
    TCC_LAUNCH_CHECK();
    TCC_HIP_CHECK(exclusive_scan(c.firstTile, c.firstTile, SW, c.firstTile + SW, c.temp, st));
    hipLaunchKernelGGL(tile_info_kernel, dim3(grid_for(SW, kThreads)), dim3(kThreads), 0, st, c.segStart,
                       c.firstTile, SW, c.tileInfo);
    TCC_LAUNCH_CHECK();
    const std::uint32_t TM = static_cast<std::uint32_t>(segment_tiles_max(E, SW));
    const std::uint64_t nCounters = static_cast<std::uint64_t>(num_bins(S)) * TM;
    if (flow32) {
        // the low digits per super-window, each pass returning at once for a
        // COO in (dst, src) order: B32 -> A32 -> B32 ...
        std::uint32_t* src = B32;
        std::uint32_t* dst = A32;
        for (const Digit& dg : plan.low) {
            SegPassArgs sa{src, dst, c.tileInfo, c.firstTile, c.segStart, E, SW, TM, dg, c.histLow, unsorted};
            const std::uint64_t nc = (1ull << dg.bits) * TM;
            hipLaunchKernelGGL(seg_hist_kernel, dim3(TM), dim3(kThreads), 0, st, sa);
            TCC_LAUNCH_CHECK();
            TCC_HIP_CHECK(exclusive_scan(c.histLow, c.histLow, nc, c.histLow + nc, c.temp, st, unsorted));
            hipLaunchKernelGGL(seg_scatter_kernel, dim3(TM), dim3(kThreads), 0, st, sa);
            TCC_LAUNCH_CHECK();
            std::swap(src, dst);
        }
    }
    TileArgs ta{};
    ta.el = sorted;
    ta.keys32 = reinterpret_cast<const std::uint32_t*>(sorted);
    // head facts: after the u32 keys in the same buffer, or in the other one
    ta.info = narrow ? reinterpret_cast<std::uint32_t*>(const_cast<std::uint64_t*>(sorted)) + E
                     : reinterpret_cast<std::uint32_t*>(sorted == c.elemA ? c.elemB : c.elemA);
    if (flow32) {
        ta.keys32 = B32;  // a COO in order: the sw passes' output
        ta.keys32Unsorted = plan.low.size() % 2 ? A32 : B32;
        ta.unsorted = unsorted;
    }
    ta.n = E;
    ta.cap = m->nnz;
    ta.keyMask = (1ull << plan.ep.kb) - 1ull;
    ta.loBits = plan.ep.loBits;
    ta.S = S;
    ta.SW = SW;
    ta.CW = CW;
    ta.segStart = c.segStart;
    ta.firstTile = c.firstTile;
    ta.tileInfo = c.tileInfo;
    ta.counters = c.counters;
    ta.TM = TM;
    ta.err = err;
    ta.wdBase = c.wdBase;
    ta.colWindowOffset = m->colWindowOffset;
    ta.occBase = c.occBase;
    ta.tileRowSlot = m->tileRowSlot;
    ta.tileBytes = reinterpret_cast<std::uint8_t*>(m->tileLocalBit);
    ta.superWindowRows = m->superWindowRows;
    ta.rowCacheSlot = m->superWindowRowCacheSlot;
    ta.cachedRowSlot = m->superWindowCachedRowSlot;

    // 3. counts, their scan, window and super-window bases
    if (narrow) hipLaunchKernelGGL(tile_count_kernel<std::uint32_t>, dim3(TM), dim3(kThreads), 0, st, ta);
    else hipLaunchKernelGGL(tile_count_kernel<std::uint64_t>, dim3(TM), dim3(kThreads), 0, st, ta);
    TCC_LAUNCH_CHECK();
    TCC_HIP_CHECK(exclusive_scan(c.counters, c.counters, nCounters, c.counters + nCounters, c.temp, st));
    hipLaunchKernelGGL(window_meta_kernel, dim3(grid_for(CW, kThreads)), dim3(kThreads), 0, st, c.counters, TM,
                       c.firstTile, S, CW, c.wdBase, c.wActive, c.wTiles);
    TCC_LAUNCH_CHECK();
    TCC_HIP_CHECK(exclusive_scan(c.wTiles, m->colWindowOffset, CW, m->colWindowOffset + CW, c.temp, st));
    hipLaunchKernelGGL(super_window_meta_kernel, dim3(grid_for(SW + 1, kThreads)), dim3(kThreads), 0, st, c.counters,
                       TM, c.firstTile, S, SW, c.occBase, m->superWindowRowOffset, m->superWindowCachedCount,
                       ws->deviceNumGroups);
    TCC_LAUNCH_CHECK();

    // 4. every output in place, then the padding rows
    if (narrow) hipLaunchKernelGGL(tile_emit_kernel<std::uint32_t>, dim3(TM), dim3(kEmitThreads), 0, st, ta);
    else hipLaunchKernelGGL(tile_emit_kernel<std::uint64_t>, dim3(TM), dim3(kEmitThreads), 0, st, ta);
    TCC_LAUNCH_CHECK();
    hipLaunchKernelGGL(padding_kernel, dim3(grid_for(CW, kThreads)), dim3(kThreads), 0, st, c.wActive,
                       m->colWindowOffset, CW, m->tileRowSlot, reinterpret_cast<std::uint8_t*>(m->tileLocalBit));
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

}  // extern "C"
