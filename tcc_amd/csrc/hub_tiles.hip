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
// Groups: G consecutive row blocks (16 degree-sorted rows each) form a
// group, and a step is a column block in which at least one of the group's
// tiles is dense.  A step holds G tile slots (zeros where the row block's
// tile is not dense), so one load of the step's 16 feature rows feeds G
// tiles: neighbouring row blocks of the core share most column blocks (at
// 114M nnz, groups of 4 cut the feature-row loads by 70% with 83% of the
// slots filled), and the feature rows, re-read once per tile from beyond L2,
// bound the kernel.
//
// Layout: rowOrder[16(G g + j) + i] = original row of row i of row block j
// of group g; group g's steps are [groupStepOffset[g], groupStepOffset[g+1]),
// step p covering column ranks 16*stepCol[p] .. +15;
// tileVals[256(G p + j) + 4l + s] = A(row l%16, column 4s + l/16) of the
// tile of row block j at step p: lane l's A operand of MFMA step s (lane l
// supplies A(i = l%16, k = l/16), B(k = l/16, j = l%16) and holds
// D(4*(l/16) + v, l%16) in register v).
//
// SpMM: the feature rows of the hub columns (ranks < hub_cols) are copied in
// rank order, TF32-rounded, into a workspace of rows padded to 64 features
// (Xh).  One wave per (unit of at most unit_steps steps of one group,
// 64-feature slice): per step G float4 of A and four float4 of Xh (four rows
// of 64 features), and 16 G MFMAs into 4 G accumulator tiles (the N tile u of
// lane l is feature 4*(l%16) + u, so one float4 of Xh feeds all four).  The
// remainder's gather runs first and fills Y; the tiles are added into it.
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "../../include/tcc_spmm_cnic.h"
#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "degree_rank.hpp"
#include "gather_ops.hpp"
#include "primitives.hpp"

namespace tcc {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr std::uint32_t kTile = 16;
constexpr std::uint32_t kTileVals = kTile * kTile;  // floats per tile
constexpr std::uint32_t kSlice = 64;                // features per wave
constexpr std::uint32_t kDefaultUnitSteps = 128;
// The remainder's gather: units of 64 blocks (config 3: 9.40-9.44 ms per
// step at 48-80 blocks, 9.58 at the 128 that tcc_bcsr's automatic choice
// gives its 4.95M blocks, 9.52 at 32; the whole phased matrix, 12.9M
// blocks, keeps 128).  Binary hybrid, its 1.41M-block remainder with the
// last chunk beside the full ones: 4.561-4.566 / 4.553-4.555 / 4.568-4.579 /
// 4.632-4.636 ms at 64 / 128 / 192 / 256 blocks (F = 602), 1.140 / 1.143 /
// 1.200 ms at 64 / 128 / 256 (F = 128).
constexpr std::uint32_t kRestUnitBlocks = 64;
constexpr std::uint32_t kMaxUnitSteps = 256;        // a unit's step columns sit one per lane, in four registers
constexpr int kColRegs = kMaxUnitSteps / 64;
constexpr std::uint32_t kDefaultMinTileNnz = 16;
constexpr std::uint32_t kDefaultGroupBlocks = 8;
// Binary tiles: steps (16 row blocks by a pair of 16-column blocks) of at
// least 40 entries, groups of 16 row blocks, units of up to 1024 sub-steps
// (the kernel reads a unit's step list 256 steps at a time, so units are
// not bound by kMaxUnitSteps).  Config 3, step ms with G = 16 on the
// sparse MFMA: 5.33 / 5.14 / 5.01 / 5.04 / 4.99 / 5.03 / 5.06 at 24 / 28 /
// 32 / 36 / 40 / 48 / 64 entries with 768-step units.  With units launched
// by size and the remainder's last chunk beside its full chunks: 4.565-4.592
// with 768-step units, 4.538-4.555 with 1024, 4.59-4.60 with 1536, 4.53-4.54
// with 2048-3072; at F = 128, 1.162-1.166 / 1.143-1.147 / 1.241 / 1.358 ms
// with 768 / 1024 / 1536 / 2048 (fewer waves); thresholds 32-40 within
// 5 us with 1024.
constexpr std::uint32_t kDefaultMinStepNnz = 40;
constexpr std::uint32_t kDefaultBinaryGroupBlocks = 16;
constexpr std::uint32_t kDefaultBinaryUnitSteps = 1024;
constexpr std::uint32_t kNoSlot = 0xFFFFFFFFu;
constexpr unsigned kThreads = 256;
constexpr std::uint32_t kXcds = 8;

// Workgroups go to the 8 XCDs round-robin (workgroup b to XCD b % 8).  The
// tile kernels deal units to XCDs the same way, unit u to XCD u % 8, and lay
// the waves of an XCD's units (their 64-feature slices, which read the same
// tiles) over that XCD's consecutive workgroups, so that one L2 holds a
// unit's tiles for all its slices.  Config 3: the split kernel's fetch fell
// from 14.0 to 10.1 GB per launch and its time from 2.04 to 1.77 ms, against
// one unit's slices on consecutive waves, which straddled XCDs.  The grid is
// kXcds * tiles_blocks_per_xcd().
__host__ __device__ inline std::uint32_t tiles_blocks_per_xcd(std::uint32_t numUnits, std::uint32_t slices) {
    const std::uint32_t unitsPerXcd = (numUnits + kXcds - 1) / kXcds;
    return (unitsPerXcd * slices + kThreads / kWave - 1) / (kThreads / kWave);
}

inline std::size_t align_up(std::size_t x) { return (x + 255) & ~std::size_t(255); }

inline bool valid_group(std::uint32_t g) { return g == 1 || g == 2 || g == 4 || g == 8; }
inline bool valid_binary_group(std::uint32_t g) { return g == 8 || g == 16; }

// bf16 halves of a TF32 value: hi = its top 16 bits (sign, exponent, 7
// mantissa bits), lo = the exact remainder (at most 3 significant bits);
// a non-finite value keeps lo = 0.  hi + lo == x for every TF32 x whose
// remainder is a normal or zero fp32 (|x| >= 2^-116).
__device__ __forceinline__ void bf16_split(float x, std::uint16_t& hi, std::uint16_t& lo) {
    const std::uint32_t b = __float_as_uint(x);
    hi = static_cast<std::uint16_t>(b >> 16);
    if ((b & 0x7F800000u) == 0x7F800000u) {
        // inf keeps lo = 0 (x - hi would be NaN); a NaN whose payload lies
        // in the low half keeps NaN through the quiet bit
        if (b & 0x007FFFFFu) hi |= 0x0040u;
        lo = 0;
        return;
    }
    const float r = x - __uint_as_float(b & 0xFFFF0000u);
    lo = static_cast<std::uint16_t>(__float_as_uint(r) >> 16);
}

// ---------------------------------------------------------------- builder

// Tile index = (group * column blocks + column block) * G + row block % G:
// the tiles of one step are adjacent.  key = tile index << 8 | (row rank %
// 16) << 4 | (column rank % 16); payload = edge.
__global__ void tile_keys_kernel(const std::uint32_t* __restrict__ row, const std::uint32_t* __restrict__ col,
                                 std::uint32_t E, const std::uint32_t* __restrict__ rowRank,
                                 const std::uint32_t* __restrict__ colRank, std::uint32_t colBlocks, std::uint32_t G,
                                 std::uint64_t* __restrict__ keys, std::uint32_t* __restrict__ perm) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint32_t rr = rowRank[row[e]], cr = colRank[col[e]];
    const std::uint32_t rb = rr / kTile;
    const std::uint64_t tile = (static_cast<std::uint64_t>(rb / G) * colBlocks + cr / kTile) * G + rb % G;
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

__device__ __forceinline__ std::uint64_t tile_index(const std::uint64_t* keys, const std::uint32_t* tileStart,
                                                    std::uint32_t t) {
    return keys[tileStart[t]] >> 8;
}

// dense[t] = tile t holds at least minNnz entries and its step (the
// stepTiles tiles of one group and step column, adjacent in the sorted
// order) at least minStepNnz; the number of dense tiles; the largest step
// column of a dense tile (+1).
__global__ void dense_tiles_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ tileStart,
                                   const std::uint32_t* __restrict__ numTiles, std::uint32_t E, std::uint32_t minNnz,
                                   std::uint32_t minStepNnz, std::uint32_t colSteps, std::uint32_t stepTiles,
                                   std::uint32_t* __restrict__ dense, std::uint32_t* __restrict__ denseCount,
                                   std::uint32_t* __restrict__ hubBlocks) {
    const std::uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    bool d = false;
    if (t < *numTiles) {
        const std::uint32_t nt = *numTiles;
        const std::uint32_t s = tileStart[t];
        const std::uint32_t e = t + 1 < nt ? tileStart[t + 1] : E;
        d = e - s >= minNnz;
        if (d && minStepNnz > e - s) {
            // the step's entries: its tiles before and after t (at most stepTiles - 1 each way)
            const std::uint64_t step = (keys[s] >> 8) / stepTiles;
            std::uint32_t first = t, end = t + 1;
            while (first > 0 && (keys[tileStart[first - 1]] >> 8) / stepTiles == step) --first;
            while (end < nt && (keys[tileStart[end]] >> 8) / stepTiles == step) ++end;
            d = (end < nt ? tileStart[end] : E) - tileStart[first] >= minStepNnz;
        }
        dense[t] = d ? 1u : 0u;
        if (d) atomicMax(hubBlocks, static_cast<std::uint32_t>((keys[s] >> 8) / stepTiles % colSteps) + 1u);
    }
    const std::uint64_t m = __ballot(d);
    if (m && __lane_id() == static_cast<unsigned>(__builtin_ctzll(m)))
        atomicAdd(denseCount, static_cast<std::uint32_t>(__builtin_popcountll(m)));
}

// stepHead[t] = tile t is dense and no earlier dense tile shares its step
// (the tiles of a step are adjacent, at most stepTiles of them); per group,
// its number of steps.
__global__ void step_heads_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ tileStart,
                                  const std::uint32_t* __restrict__ numTiles, const std::uint32_t* __restrict__ dense,
                                  std::uint32_t stepTiles, std::uint32_t colSteps, std::uint32_t* __restrict__ stepHead,
                                  std::uint32_t* __restrict__ groupSteps) {
    const std::uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= *numTiles) return;
    std::uint32_t head = 0;
    if (dense[t]) {
        const std::uint64_t step = tile_index(keys, tileStart, t) / stepTiles;
        head = 1;
        for (std::uint32_t b = t; b > 0; --b) {
            if (tile_index(keys, tileStart, b - 1) / stepTiles != step) break;
            if (dense[b - 1]) {
                head = 0;
                break;
            }
        }
        if (head) atomicAdd(&groupSteps[step / colSteps], 1u);
    }
    stepHead[t] = head;
}

// Per dense tile: its slot (step * stepTiles + tile % stepTiles) and, for
// step heads, the step's column (a 16-column block, or a pair of them for
// binary tiles).
__global__ void tile_slots_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ tileStart,
                                  const std::uint32_t* __restrict__ numTiles, const std::uint32_t* __restrict__ dense,
                                  const std::uint32_t* __restrict__ stepHead, const std::uint32_t* __restrict__ stepPos,
                                  std::uint32_t stepTiles, std::uint32_t colSteps, std::uint32_t* __restrict__ slot,
                                  std::uint32_t* __restrict__ stepCol) {
    const std::uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= *numTiles || !dense[t]) return;
    const std::uint64_t tile = tile_index(keys, tileStart, t);
    const std::uint32_t step = stepPos[t] + stepHead[t] - 1;  // heads up to and including t, minus one
    slot[t] = step * stepTiles + static_cast<std::uint32_t>(tile % stepTiles);
    if (stepHead[t]) stepCol[step] = static_cast<std::uint32_t>(tile / stepTiles % colSteps);
}

// Per edge: 1 if it stays in the sparse remainder.
__global__ void rest_flags_kernel(const std::uint32_t* __restrict__ flags, const std::uint32_t* __restrict__ pos,
                                  const std::uint32_t* __restrict__ dense, std::uint32_t E,
                                  std::uint32_t* __restrict__ rest) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e < E) rest[e] = dense[pos[e] + flags[e] - 1] ? 0u : 1u;
}

__global__ void units_per_group_kernel(const std::uint32_t* __restrict__ groupSteps, std::uint32_t NG,
                                       std::uint32_t unitSteps, std::uint32_t* __restrict__ units) {
    const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g < NG) units[g] = (groupSteps[g] + unitSteps - 1) / unitSteps;
}

// Dense tiles' entries into their slots (TF32-rounded values in the
// A-operand order, or pattern bits), the others into the remainder COO.
__global__ void place_entries_kernel(const std::uint64_t* __restrict__ keys, const std::uint32_t* __restrict__ perm,
                                     std::uint32_t E, const std::uint32_t* __restrict__ flags,
                                     const std::uint32_t* __restrict__ pos, const std::uint32_t* __restrict__ dense,
                                     const std::uint32_t* __restrict__ slot, const std::uint32_t* __restrict__ restPos,
                                     const std::uint32_t* __restrict__ row, const std::uint32_t* __restrict__ col,
                                     const float* __restrict__ val, float* __restrict__ tileVals,
                                     std::uint32_t format, std::uint32_t G, std::uint32_t* __restrict__ tileMasks,
                                     std::uint32_t* __restrict__ restRow, std::uint32_t* __restrict__ restCol,
                                     float* __restrict__ restVal) {
    const std::uint32_t e = blockIdx.x * blockDim.x + threadIdx.x;
    if (e >= E) return;
    const std::uint32_t t = pos[e] + flags[e] - 1;
    const std::uint32_t src = perm[e];
    const float v = val ? val[src] : 1.0f;
    if (dense[t]) {
        const std::uint32_t i = static_cast<std::uint32_t>(keys[e] >> 4) & 15u, j = static_cast<std::uint32_t>(keys[e]) & 15u;
        if (format == TCC_TILES_BINARY) {
            // the step's raw bits (binary_encode_kernel's input): 32 G bytes
            // per 16-column half h of the step, byte l*(G/2) + rb/2 with
            // l = 16*(rb%2) + i + 32*(j/8), bit j%8
            const std::uint32_t step = slot[t] / (2 * G), q = slot[t] % (2 * G), h = q / G, rb = q % G;
            const std::uint64_t byte = (2ull * step + h) * G * 32 + (16 * (rb % 2) + i + 32 * (j / 8)) * (G / 2) + rb / 2;
            atomicOr(&tileMasks[byte / 4], 1u << (8 * (byte % 4) + j % 8));
        } else if (format == TCC_TILES_BF16X2) {
            // bf16 tile: hi[i][j] at 2(16i + j) bytes, lo 512 bytes further
            std::uint16_t hi, lo;
            bf16_split(tf32_rna(v), hi, lo);
            std::uint16_t* tile = reinterpret_cast<std::uint16_t*>(tileVals + static_cast<std::uint64_t>(slot[t]) * kTileVals);
            tile[16 * i + j] = hi;
            tile[256 + 16 * i + j] = lo;
        } else {
            const std::uint32_t lane = i + 16 * (j % 4), step = j / 4;
            tileVals[static_cast<std::uint64_t>(slot[t]) * kTileVals + 4 * lane + step] = tf32_rna(v);
        }
    } else {
        const std::uint32_t p = restPos[e];
        restRow[p] = row[src];
        restCol[p] = col[src];
        if (restVal) restVal[p] = v;
    }
}

// ---- binary tiles: the pattern as operands of the 2:4 sparse MFMA
//
// v_smfmac_f32_32x32x32_f16 multiplies a 32x32 A held as two values of each
// group of four consecutive columns (8 values a lane and 2-bit positions)
// by a dense 32x32 B.  A binary step covers 32 columns (two 16-column
// blocks, h = 0 and 1) of G/2 32-row tiles; lane l of the wave supplies
// row l%32 of each tile and, with c = l/32, columns 8c..8c+7 of both
// halves: value slots 2k and 2k+1 of the lane hold the entries of its
// nibble k (k = 0, 1: columns 8c + 4k..+3 of half 0; k = 2, 3: columns
// 8c + 4(k-2)..+3 of half 1), and B's lane l holds the 16 columns of half
// c for feature l%32.  A nibble with more than two entries does not fit:
// such a step takes a second layer, the same columns with each nibble's
// entries past its lowest two.

// Lane bytes of a step's raw half h (G/2 bytes: one per 32-row tile).
__device__ __forceinline__ std::uint64_t raw_lane_bytes(const std::uint32_t* raw, std::uint32_t G, std::uint64_t step,
                                                        std::uint32_t h, unsigned lane) {
    const std::uint32_t* p = raw + ((2 * step + h) * G * 32 + lane * (G / 2)) / 4;
    if (G != 16) return *p;
    const vu2 v = load_global<vu2>(p);
    return v.x | static_cast<std::uint64_t>(v.y) << 32;
}

// Nibbles of x holding more than two set bits.
__device__ __forceinline__ bool crowded_nibble(std::uint64_t x) {
    std::uint64_t c = x - ((x >> 1) & 0x5555555555555555ull);
    c = (c & 0x3333333333333333ull) + ((c >> 2) & 0x3333333333333333ull);  // per-nibble counts, 0..4
    return ((c + 0x1111111111111111ull) & 0xCCCCCCCCCCCCCCCCull) != 0;      // count + 1 >= 4
}

// layers[s] = 2 when a nibble of step s holds more than two entries, else 1
// (one wave per step).
__global__ void binary_layers_kernel(const std::uint32_t* __restrict__ raw, std::uint32_t NS, std::uint32_t G,
                                     std::uint32_t* __restrict__ layers) {
    const std::uint64_t s = (static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
    if (s >= NS) return;
    const unsigned lane = __lane_id();
    const bool crowded = crowded_nibble(raw_lane_bytes(raw, G, s, 0, lane)) || crowded_nibble(raw_lane_bytes(raw, G, s, 1, lane));
    const std::uint64_t any = __ballot(crowded);
    if (lane == 0) layers[s] = any ? 2u : 1u;
}

// subOffset[g] = first sub-step of group g (g <= NG); groupSub[g] = its
// sub-steps (steps and second layers).
__global__ void sub_offsets_kernel(const std::uint32_t* __restrict__ stepOffset, const std::uint32_t* __restrict__ subPos,
                                   std::uint32_t NG, std::uint32_t* __restrict__ subOffset,
                                   std::uint32_t* __restrict__ groupSub) {
    const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g > NG) return;
    subOffset[g] = subPos[stepOffset[g]];
    if (g < NG) groupSub[g] = subPos[stepOffset[g + 1]] - subPos[stepOffset[g]];
}

// Two value slots of one nibble's entries in a layer (layer 0: the lowest
// two set bits, layer 1: the rest): value bits (slot 0 in bit 0) and the
// slots' positions (2 bits each, slot 0 low).  Positions increase; a slot
// without an entry holds 0 and points at an unused position.
__device__ __forceinline__ void encode_nibble(unsigned nib, int layer, unsigned& vals, unsigned& pos) {
    const unsigned l1 = nib & (0u - nib), r1 = nib & ~l1, l2 = r1 & (0u - r1);
    const unsigned sel = layer ? nib & ~(l1 | l2) : (l1 | l2);
    const int n = __builtin_popcount(sel);
    if (n == 2) {
        const unsigned p0 = static_cast<unsigned>(__builtin_ctz(sel)), p1 = static_cast<unsigned>(__builtin_ctz(sel & (sel - 1)));
        vals = 3u;
        pos = p0 | p1 << 2;
    } else if (n == 1) {
        const unsigned p = static_cast<unsigned>(__builtin_ctz(sel));
        vals = p < 3 ? 1u : 2u;
        pos = p < 3 ? (p | 3u << 2) : (2u | 3u << 2);
    } else {
        vals = 0u;
        pos = 0u | 1u << 2;
    }
}

// Sub-step records (one wave per step): the step's layers at sub-steps
// subPos[s].., each 96 G bytes: lane l's G/2 value-mask bytes at l*(G/2)
// (byte t: tile t, bit j: value slot j is 1.0), then at 32 G + l*G the
// 16-bit positions of tile t at byte 2t (slot j in bits 2j..2j+1).
__global__ void binary_encode_kernel(const std::uint32_t* __restrict__ raw, std::uint32_t NS, std::uint32_t G,
                                     const std::uint32_t* __restrict__ subPos, const std::uint32_t* __restrict__ stepColIn,
                                     std::uint32_t* __restrict__ out, std::uint32_t* __restrict__ stepCol) {
    const std::uint64_t s = (static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
    if (s >= NS) return;
    const unsigned lane = __lane_id();
    const std::uint64_t w0 = raw_lane_bytes(raw, G, s, 0, lane), w1 = raw_lane_bytes(raw, G, s, 1, lane);
    const std::uint32_t sub0 = subPos[s], layers = subPos[s + 1] - sub0;
    const std::uint32_t T = G / 2;
    for (std::uint32_t L = 0; L < layers; ++L) {
        std::uint64_t masks = 0;
        std::uint32_t idx[8] = {};
        for (std::uint32_t t = 0; t < T; ++t) {
            const unsigned b0 = static_cast<unsigned>(w0 >> (8 * t)) & 0xFFu, b1 = static_cast<unsigned>(w1 >> (8 * t)) & 0xFFu;
            const unsigned nib[4] = {b0 & 15u, b0 >> 4, b1 & 15u, b1 >> 4};
            unsigned m = 0, p = 0;
            for (int k = 0; k < 4; ++k) {
                unsigned v, q;
                encode_nibble(nib[k], static_cast<int>(L), v, q);
                m |= v << (2 * k);
                p |= q << (4 * k);
            }
            masks |= static_cast<std::uint64_t>(m) << (8 * t);
            idx[t] = p;
        }
        std::uint32_t* rec = out + (static_cast<std::uint64_t>(sub0) + L) * 24 * G;
        std::uint32_t* mp = rec + lane * (G / 8);
        std::uint32_t* ip = rec + 8 * G + lane * (G / 4);
        if (G == 16) {
            *reinterpret_cast<vu2*>(mp) = vu2{static_cast<std::uint32_t>(masks), static_cast<std::uint32_t>(masks >> 32)};
            *reinterpret_cast<vu4*>(ip) = vu4{idx[0] | idx[1] << 16, idx[2] | idx[3] << 16, idx[4] | idx[5] << 16,
                                              idx[6] | idx[7] << 16};
        } else {
            *mp = static_cast<std::uint32_t>(masks);
            *reinterpret_cast<vu2*>(ip) = vu2{idx[0] | idx[1] << 16, idx[2] | idx[3] << 16};
        }
        if (lane == 0) stepCol[sub0 + L] = stepColIn[s];
    }
}

// units[3u .. 3u+2] = group, first step, end step.
__global__ void group_units_kernel(const std::uint32_t* __restrict__ groupStepOffset,
                                   const std::uint32_t* __restrict__ unitFirst, std::uint32_t NG, std::uint32_t unitSteps,
                                   std::uint32_t* __restrict__ units) {
    const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= NG) return;
    const std::uint32_t s0 = groupStepOffset[g], s1 = groupStepOffset[g + 1];
    for (std::uint32_t k = 0; unitFirst[g] + k < unitFirst[g + 1]; ++k) {
        const std::uint64_t u = 3ull * (unitFirst[g] + k);
        units[u] = g;
        units[u + 1] = s0 + k * unitSteps;
        units[u + 2] = min(s0 + (k + 1) * unitSteps, s1);
    }
}

// Sort keys of the launch order: the column block of each unit's first step
// (a unit has at least one step), the unit index as payload.  With
// bySize, the units come in buckets of 128 steps, the largest first, and by
// column within a bucket: a long unit launched last would hold the grid's
// tail (binary tiles, config 3: 4.76 -> 4.68 ms per hybrid step).
constexpr std::uint32_t kOrderBucketSteps = 128;
constexpr std::uint32_t kOrderBuckets = 1u << 16;

__global__ void unit_order_keys_kernel(const std::uint32_t* __restrict__ units, const std::uint32_t* __restrict__ stepCol,
                                       std::uint32_t NU, bool bySize, unsigned colBits,
                                       std::uint64_t* __restrict__ keys, std::uint32_t* __restrict__ order) {
    const std::uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u >= NU) return;
    const std::uint32_t first = units[3ull * u + 1], end = units[3ull * u + 2];
    const std::uint64_t bucket = min((end - first) / kOrderBucketSteps, kOrderBuckets - 1);
    keys[u] = (bySize ? (kOrderBuckets - 1 - bucket) << colBits : 0) | stepCol[first];
    order[u] = u;
}

// Units of shared groups (groups held by more than one unit) get
// consecutive partial-sum slots in unit order: flags per group and per unit
// for two scans, then the slots and the list of shared groups.
__global__ void shared_groups_kernel(const std::uint32_t* __restrict__ unitFirst, std::uint32_t NG,
                                     std::uint32_t* __restrict__ groupShared) {
    const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g < NG) groupShared[g] = unitFirst[g + 1] - unitFirst[g] > 1 ? 1u : 0u;
}

__global__ void shared_units_kernel(const std::uint32_t* __restrict__ units, std::uint32_t NU,
                                    const std::uint32_t* __restrict__ groupShared, std::uint32_t* __restrict__ unitShared) {
    const std::uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u < NU) unitShared[u] = groupShared[units[3ull * u]];
}

__global__ void partial_slots_kernel(std::uint32_t NU, const std::uint32_t* __restrict__ unitShared,
                                     const std::uint32_t* __restrict__ unitPos, std::uint32_t* __restrict__ unitPartial) {
    const std::uint32_t u = blockIdx.x * blockDim.x + threadIdx.x;
    if (u < NU) unitPartial[u] = unitShared[u] ? unitPos[u] : kNoSlot;
}

// sharedGroups[3s .. 3s+2] = group, slot of its first unit, its units
__global__ void shared_group_list_kernel(const std::uint32_t* __restrict__ unitFirst, std::uint32_t NG,
                                         const std::uint32_t* __restrict__ groupShared,
                                         const std::uint32_t* __restrict__ groupPos,
                                         const std::uint32_t* __restrict__ unitPos,
                                         std::uint32_t* __restrict__ sharedGroups) {
    const std::uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= NG || !groupShared[g]) return;
    const std::uint64_t s = 3ull * groupPos[g];
    sharedGroups[s] = g;
    sharedGroups[s + 1] = unitPos[unitFirst[g]];
    sharedGroups[s + 2] = unitFirst[g + 1] - unitFirst[g];
}

// out[s] = scale of row rowOrder[s] (0 for the slots past the last row)
__global__ void ordered_scale_kernel(const std::uint32_t* __restrict__ rowOrder, std::uint32_t n,
                                     const float* __restrict__ scale, float* __restrict__ out) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const std::uint32_t r = rowOrder[i];
    out[i] = r != TCC_SWTCF_INVALID_ROW_SLOT ? scale[r] : 0.0f;
}

// out[i] = in[i] for i < n, 0 up to `padded`
__global__ void padded_copy_kernel(const float* __restrict__ in, std::uint32_t n, std::uint32_t padded,
                                   float* __restrict__ out) {
    const std::uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < padded) out[i] = i < n ? in[i] : 0.0f;
}

// A BCSR's entries as a COO (tcc_hybrid_from_bcsr): block b's window is
// the last w with rowWindowOffset[w] <= b; its valid bits are those whose
// column slot names a column (< numCols) and whose row is < numRows.
__device__ __forceinline__ std::uint32_t block_window(const std::uint32_t* winOffset, std::uint32_t W, std::uint32_t b) {
    std::uint32_t lo = 0, hi = W;  // winOffset[lo] <= b < winOffset[hi]
    while (hi - lo > 1) {
        const std::uint32_t mid = lo + (hi - lo) / 2;
        if (winOffset[mid] <= b) lo = mid;
        else hi = mid;
    }
    return lo;
}

__device__ __forceinline__ std::uint64_t block_valid_bits(const tcc_bcsr& A, std::uint32_t b, std::uint32_t w) {
    std::uint64_t colMask = 0, rowMask = 0;
#pragma unroll
    for (int c = 0; c < 8; ++c)
        if (A.sparseA2B[8ull * b + c] < A.num_cols) colMask |= 0x0101010101010101ull << c;
#pragma unroll
    for (int r = 0; r < 8; ++r)
        if (8ull * w + r < A.num_rows) rowMask |= 0xFFull << (8 * r);
    return A.tcLocalBit[b] & colMask & rowMask;
}

__global__ void bcsr_entry_counts_kernel(tcc_bcsr A, std::uint32_t* __restrict__ counts) {
    const std::uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= A.num_TCBlocks) return;
    const std::uint32_t w = block_window(A.rowWindowOffset, A.num_rowWindows, b);
    counts[b] = static_cast<std::uint32_t>(__popcll(block_valid_bits(A, b, w)));
}

__global__ void bcsr_expand_kernel(tcc_bcsr A, const std::uint32_t* __restrict__ offset, bool values,
                                   std::uint32_t* __restrict__ row, std::uint32_t* __restrict__ col,
                                   float* __restrict__ val) {
    const std::uint32_t b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= A.num_TCBlocks) return;
    const std::uint32_t w = block_window(A.rowWindowOffset, A.num_rowWindows, b);
    const std::uint64_t stored = A.tcLocalBit[b];
    std::uint64_t m = block_valid_bits(A, b, w);
    std::uint32_t k = offset[b];
    while (m) {
        const unsigned i = static_cast<unsigned>(__builtin_ctzll(m));
        m &= m - 1;
        row[k] = 8 * w + i / 8;
        col[k] = A.sparseA2B[8ull * b + i % 8];
        // values follow the stored bits in ascending order (data[tcOffset[b] + rank])
        if (values) val[k] = A.data[A.tcOffset[b] + __popcll(stored & ((1ull << i) - 1ull))];
        ++k;
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

// Xh[r][f] = TF32(X[hubColOrder[r]][f]) for r < hubCols and f < F, 0 for
// the other f < ldh and the rows up to hubRows (the last column block's
// ranks past the last column); one thread per 4 features (ldh is a
// multiple of 64).
__global__ void hub_rows_kernel(const float* __restrict__ X, std::uint32_t F, const std::uint32_t* __restrict__ order,
                                std::uint32_t hubCols, std::uint32_t hubRows, std::uint32_t ldh, bool vec,
                                float* __restrict__ Xh) {
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::uint32_t q = ldh / 4;
    const std::uint32_t r = static_cast<std::uint32_t>(i / q), f = 4 * static_cast<std::uint32_t>(i % q);
    if (r >= hubRows) return;
    f32x4 v = {0.0f, 0.0f, 0.0f, 0.0f};
    if (r >= hubCols) {
        *reinterpret_cast<f32x4*>(Xh + static_cast<std::uint64_t>(r) * ldh + f) = v;
        return;
    }
    const float* x = X + static_cast<std::uint64_t>(order[r]) * F + f;
    if (vec && f + 4 <= F) {
        v = load_global<vf4>(x);
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (f + u < F) v[u] = x[u];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = tf32_rna(v[u]);
    *reinterpret_cast<f32x4*>(Xh + static_cast<std::uint64_t>(r) * ldh + f) = v;
}

struct TileArgs {
    const std::uint32_t* rowOrder;
    const std::uint32_t* groupStepOffset;
    const std::uint32_t* stepCol;
    const float* tileVals;
    const std::uint32_t* tileMasks;  // binary tiles
    const float* rowScale;           // binary tiles: row scales in rowOrder's order, or null
    const std::uint32_t* units;
    const std::uint32_t* unitPartial;   // partial-sum slot of each unit (kNoSlot: it holds its group)
    const std::uint32_t* sharedGroups;  // (group, first slot, units) of each shared group
    const float* Xh;
    std::uint32_t ldh;  // Xh row stride (a multiple of 64)
    float* Y;
    float* partials;    // [num_partial_units][16 G][ldh]: sums of the units of shared groups
    std::uint32_t zeroStep;  // num_steps: a step of G zero tiles after the last
    std::uint32_t F;
    std::uint32_t numUnits;
    std::uint32_t slices;    // feature slices per unit (ldh / features per wave)
    const std::uint32_t* unitOrder;  // launch order of the units, or null
    // Binary tiles over half records (hub_rows_half_kernel): per (column
    // block, slice) 1 where Xs holds fp16 values, and per slice the factor
    // 2^-e that undoes the slice's scale; null: bf16 records throughout.
    const unsigned char* halfFlags;
    const float* sliceDown;
    // Binary tiles: store the sums into Y instead of adding them (the
    // hybrid's remainder adds into Y after; hub_zero_rows_kernel zeroes the
    // rows no unit writes).
    int storeY;
    std::uint32_t zeroCol;  // binary tiles: the column-block pair of zeros in Xs (the zero step's)
};

// This wave's unit and 64-feature slice (unit >= numUnits: no work).  The
// i-th unit launched is unitOrder[i]: units sorted by the column block of
// their first step, so that the units running at one time read about the
// same hub rows (config 3: 18% less fetched, 1.77 -> 1.69 ms).
__device__ __forceinline__ void tile_wave(const TileArgs& a, std::uint32_t& unit, std::uint32_t& slice) {
    const std::uint32_t wx = blockIdx.x / kXcds * (kThreads / kWave) +
                             static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave)));
    const std::uint32_t j = wx / a.slices;
    slice = wx - j * a.slices;
    unit = j * kXcds + blockIdx.x % kXcds;
    if (a.unitOrder && unit < a.numUnits) unit = a.unitOrder[unit];
}

// One step's operands for one wave: A of the G tiles (lane l: A(l%16,
// 4s + l/16), s = 0..3) and four 4-row steps of Xh (lane l: row 4s + l/16,
// features 4(l%16)..+3).
template <int G>
struct StepOperands {
    f32x4 a[G];
    f32x4 b[4];
};

// Y[row][f..f+3] += s (features below F only).
__device__ __forceinline__ void add_quad(float* row, std::uint32_t f, std::uint32_t F, bool vec, const f32x4& s,
                                         bool store = false) {
    if (!row || f >= F) return;
    float* out = row + f;
    if (vec) {
        f32x4 y = store ? f32x4{0.0f, 0.0f, 0.0f, 0.0f} : load_global<vf4>(out);
        y += s;
        *reinterpret_cast<f32x4*>(out) = y;
    } else {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            if (f + u < F) out[u] = store ? s[u] : out[u] + s[u];
    }
}

// One wave per (unit of at most 256 steps of one group, 64-feature slice),
// the slices of a unit on one XCD (tile_wave), so that they read the same
// tiles through one L2.  The unit's step columns sit one per lane and are read with
// readlane; operands are loaded NS - 1 steps ahead into a ring of NS
// stages, every load unconditional: loads complete in order, so a
// conditional load, a copy between stages or a branch out of the ring would
// make the wave wait for the newest one; the last trip's steps past the
// unit's end multiply the zero step's A instead.  A group
// held by one unit adds its sums into Y; the units of a shared group store
// theirs in `partials` for hub_reduce_kernel (no atomics, and a sum order
// that does not depend on scheduling).
// The unit's step columns, one per lane: register k holds steps 64k..64k+63.
__device__ __forceinline__ void load_step_cols(const std::uint32_t* stepCol, std::uint32_t p0, std::uint32_t last,
                                               int (&cols)[kColRegs]) {
#pragma unroll
    for (int k = 0; k < kColRegs; ++k) cols[k] = static_cast<int>(stepCol[min(p0 + 64u * k + __lane_id(), last)]);
}

// As load_step_cols, with bit 31 of each step's entry set where the step's
// column block holds half records for this wave's slice (flags non-null).
__device__ __forceinline__ void load_step_cols_flagged(const std::uint32_t* stepCol, std::uint32_t p0,
                                                       std::uint32_t last, int (&cols)[kColRegs],
                                                       const unsigned char* flags, std::uint32_t slices,
                                                       std::uint32_t slice) {
    load_step_cols(stepCol, p0, last, cols);
    if (!flags) return;
#pragma unroll
    for (int k = 0; k < kColRegs; ++k) {
        const std::uint32_t c = static_cast<std::uint32_t>(cols[k]);
        if (flags[static_cast<std::uint64_t>(c) * slices + slice]) cols[k] = static_cast<int>(c | 0x80000000u);
    }
}

// Column block of step q of the unit (q uniform): lane q % 64 of register q / 64.
__device__ __forceinline__ std::uint32_t step_col(const int (&cols)[kColRegs], std::uint32_t q) {
    int c = __builtin_amdgcn_readlane(cols[0], static_cast<int>(q & 63u));
#pragma unroll
    for (int k = 1; k < kColRegs; ++k) {
        const int ck = __builtin_amdgcn_readlane(cols[k], static_cast<int>(q & 63u));
        c = (q >> 6) == static_cast<std::uint32_t>(k) ? ck : c;
    }
    return static_cast<std::uint32_t>(c);
}

template <int G, int NS>
__global__ void __launch_bounds__(kThreads) hub_tiles_kernel(TileArgs a) {
    const unsigned lane = __lane_id();
    std::uint32_t unit, slice;
    tile_wave(a, unit, slice);
    if (unit >= a.numUnits) return;
    const std::uint32_t g = a.units[3ull * unit], p0 = a.units[3ull * unit + 1], p1 = a.units[3ull * unit + 2];
    if (p0 >= p1) return;
    const std::uint32_t pslot = a.unitPartial[unit];
    const bool shared = pslot != kNoSlot;
    const std::uint32_t f0 = slice * kSlice;
    const unsigned li = lane & 15u, lk = lane >> 4;
    const std::uint32_t last = p1 - 1;
    int cols[kColRegs];
    load_step_cols(a.stepCol, p0, last, cols);
    // this lane's B element offset in a 4-row step: row lk, features 4*li..+3
    const float* xb = a.Xh + static_cast<std::uint64_t>(lk) * a.ldh + f0 + 4 * li;
    const float* av = a.tileVals + 4 * lane;

    // step p's operands; past the unit's end (the ring's tail) A comes from
    // the zero step, so the products add nothing
    auto load = [&](std::uint32_t p, StepOperands<G>& o) {
        const std::uint32_t pa = p <= last ? p : a.zeroStep;
        const std::uint32_t col = step_col(cols, min(p, last) - p0);
#pragma unroll
        for (int j = 0; j < G; ++j)
            o.a[j] = load_global<vf4>(av + (static_cast<std::uint64_t>(pa) * G + j) * kTileVals);
        const float* rb = xb + static_cast<std::uint64_t>(col) * kTile * a.ldh;
#pragma unroll
        for (int s = 0; s < 4; ++s) o.b[s] = load_global<vf4>(rb + static_cast<std::uint64_t>(4 * s) * a.ldh);
    };
    f32x4 acc[G][4];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[j][u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto mma = [&](const StepOperands<G>& o) {
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int u = 0; u < 4; ++u)
                    acc[j][u] = __builtin_amdgcn_mfma_f32_16x16x4f32(o.a[j][s], o.b[s][u], acc[j][u], 0, 0, 0);
    };

    StepOperands<G> ring[NS];
#pragma unroll
    for (int k = 0; k < NS - 1; ++k) {
        load(p0 + k, ring[k]);
        __builtin_amdgcn_sched_barrier(0);  // stage k's loads before stage k+1's
    }
    for (std::uint32_t p = p0; p < p1; p += NS) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            load(p + k + NS - 1, ring[(k + NS - 1) % NS]);
            // keep the loads ahead of the products (the scheduler would
            // sink them next to their use to save registers)
            __builtin_amdgcn_sched_barrier(0);
            mma(ring[k]);
        }
    }

    // D(4*lk + v, li) of N tile u of row block j: row 16j + 4*lk + v of the
    // group, feature f0 + 4*li + u.
    const std::uint32_t f = f0 + 4 * li;
    if (shared) {
        float* base = a.partials + (static_cast<std::uint64_t>(pslot) * G * kTile + 4 * lk) * a.ldh + f;
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                *reinterpret_cast<f32x4*>(base + static_cast<std::uint64_t>(16 * j + v) * a.ldh) =
                    f32x4{acc[j][0][v], acc[j][1][v], acc[j][2][v], acc[j][3][v]};
        return;
    }
    // rows 16j + 4lk .. +3 of the group: one 16-byte load per row block,
    // then every Y quad loaded before any is stored
    vu4 rows[G];
#pragma unroll
    for (int j = 0; j < G; ++j)
        rows[j] = load_global<vu4>(a.rowOrder + static_cast<std::uint64_t>(g) * G * kTile + 16 * j + 4 * lk);
    const bool vec = a.F % 4 == 0 && (reinterpret_cast<std::uintptr_t>(a.Y) & 15u) == 0;
    if (vec) {
        f32x4 y[G][4];
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const bool live = rows[j][v] != TCC_SWTCF_INVALID_ROW_SLOT && f < a.F;
                y[j][v] = live ? load_global<vf4>(a.Y + static_cast<std::uint64_t>(rows[j][v]) * a.F + f)
                               : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (rows[j][v] != TCC_SWTCF_INVALID_ROW_SLOT && f < a.F)
                    *reinterpret_cast<f32x4*>(a.Y + static_cast<std::uint64_t>(rows[j][v]) * a.F + f) =
                        y[j][v] + f32x4{acc[j][0][v], acc[j][1][v], acc[j][2][v], acc[j][3][v]};
        return;
    }
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            if (rows[j][v] == TCC_SWTCF_INVALID_ROW_SLOT) continue;
            add_quad(a.Y + static_cast<std::uint64_t>(rows[j][v]) * a.F, f, a.F, false,
                     f32x4{acc[j][0][v], acc[j][1][v], acc[j][2][v], acc[j][3][v]});
        }
}

// Split tiles (TCC_TILES_BF16X2).  A TF32 value is exactly hi + lo with
// both bf16, and a bf16 product is exact in fp32, so a·x = ah·xh + ah·xl +
// al·xh + al·xl accumulates in fp32 like the fp32 MFMA of TF32 operands, at
// four bf16 products per TF32 one: v_mfma_f32_16x16x32_bf16 runs 16x the
// fp32 MFMA's rate (D[i][j] = sum_q sum_e A[lane i+16q][e] B[lane j+16q][e]
// over lane groups q = l/16 and elements e, checked on the GPU).  Xs holds
// the hub rows transposed per column block: Xs[cb][f] = 16 hi then 16 lo
// bf16 of rows 16cb..16cb+15 (64 bytes), so that a lane's 8 values of one
// k-half are one 16-byte load.
// With colScale (binary tiles), column c's row is TF32(colScale[c] * X[c]).
__global__ void hub_rows_split_kernel(const float* __restrict__ X, std::uint32_t F,
                                      const std::uint32_t* __restrict__ order, std::uint32_t hubCols,
                                      std::uint32_t hubRows, std::uint32_t ldh, const float* __restrict__ colScale,
                                      std::uint16_t* __restrict__ Xs) {
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::uint32_t cb = static_cast<std::uint32_t>(i / ldh), f = static_cast<std::uint32_t>(i % ldh);
    if (cb >= hubRows / kTile) return;
    // the 16 rows' values loaded before any is used (clamped indices,
    // zeroed after): loads under their bounds branches were each waited for
    std::uint32_t src[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) src[k] = order[min(cb * kTile + k, hubCols > 0 ? hubCols - 1 : 0u)];
    const std::uint32_t fc = min(f, F > 0 ? F - 1 : 0u);
    float x[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) x[k] = X[static_cast<std::uint64_t>(src[k]) * F + fc];
    if (colScale) {
#pragma unroll
        for (int k = 0; k < 16; ++k) x[k] *= colScale[src[k]];
    }
    vu4 hi[2], lo[2];
#pragma unroll
    for (int k = 0; k < 16; k += 2) {
        std::uint16_t h0 = 0, l0 = 0, h1 = 0, l1 = 0;
        const std::uint32_t r = cb * kTile + k;
        if (f < F && r < hubCols) bf16_split(tf32_rna(x[k]), h0, l0);
        if (f < F && r + 1 < hubCols) bf16_split(tf32_rna(x[k + 1]), h1, l1);
        hi[k / 8][(k % 8) / 2] = static_cast<std::uint32_t>(h0) | static_cast<std::uint32_t>(h1) << 16;
        lo[k / 8][(k % 8) / 2] = static_cast<std::uint32_t>(l0) | static_cast<std::uint32_t>(l1) << 16;
    }
    vu4* out = reinterpret_cast<vu4*>(Xs + (static_cast<std::uint64_t>(cb) * ldh + f) * 32);
    out[0] = hi[0];
    out[1] = hi[1];
    out[2] = lo[0];
    out[3] = lo[1];
}

// Half records for binary tiles.  The hub rows' TF32 values x (of
// colScale[c] * X[c]) are multiplied by 2^e, one e per slice of W features
// (a wave's slice), chosen from the slice's largest finite |x| over the hub
// rows so that it maps into [2^15, 2^16): e = 15 - E for a largest magnitude
// in [2^E, 2^(E+1)), at least 0 and at most 126 (0 for a slice without
// one).  A (column block, slice) record set whose every 2^e x is an fp16
// value (no finite value overflows; a value below 2^(-14-e) must lie on the
// fp16 grid) holds those fp16 values in its hi slots, and its flag is 1;
// any other keeps the exact bf16 halves of 2^e x.  Both are exact, and the
// tile kernel multiplies its sums by 2^-e.
//
// hub_absmax_kernel: thread i takes 4 consecutive features of hub row
// i / quads (the flat (row, quad) range cut into one stretch per workgroup,
// walked 256 quads at a time), the workgroup's largest finite |x| bits per
// slice gathered with LDS atomics, then added by atomicMax into row
// blockIdx.x % kPackSliceMaxRows of partial[kPackSliceMaxRows][slices] (zeroed
// first; the remainder's TF32 pack fills the same rows over all columns
// when a hybrid runs one).  hub_scale_kernel (one workgroup per slice)
// reduces the rows into 2^e and 2^-e.
__global__ void __launch_bounds__(kThreads) hub_absmax_kernel(const float* __restrict__ X, std::uint32_t F,
                                                             const std::uint32_t* __restrict__ order,
                                                             std::uint32_t hubCols, const float* __restrict__ colScale,
                                                             std::uint32_t W, std::uint32_t slices,
                                                             std::uint32_t* __restrict__ partial) {
    extern __shared__ std::uint32_t smax[];
    for (std::uint32_t s = threadIdx.x; s < slices; s += blockDim.x) smax[s] = 0;
    __syncthreads();
    const std::uint32_t quads = (F + 3) / 4;
    const std::uint64_t total = static_cast<std::uint64_t>(hubCols) * quads;
    const std::uint64_t per = (total + gridDim.x - 1) / gridDim.x;
    const std::uint64_t begin = per * blockIdx.x, end = min(total, begin + per);
    // four quads a thread at a time, their loads issued together
    constexpr std::uint32_t kItems = 4;
    for (std::uint64_t i0 = begin + threadIdx.x; i0 < end; i0 += kItems * blockDim.x) {
        std::uint32_t src[kItems], f[kItems];
#pragma unroll
        for (std::uint32_t j = 0; j < kItems; ++j) {
            const std::uint64_t i = min(i0 + j * blockDim.x, end - 1);
            f[j] = 4 * static_cast<std::uint32_t>(i % quads);
            src[j] = order[i / quads];
        }
        float v[kItems][4], sc[kItems];
#pragma unroll
        for (std::uint32_t j = 0; j < kItems; ++j) {
            sc[j] = colScale ? colScale[src[j]] : 1.0f;
            const float* x = X + static_cast<std::uint64_t>(src[j]) * F;
#pragma unroll
            for (std::uint32_t k = 0; k < 4; ++k) v[j][k] = x[min(f[j] + k, F - 1)];
        }
#pragma unroll
        for (std::uint32_t j = 0; j < kItems; ++j) {
            if (i0 + j * blockDim.x >= end) break;
            std::uint32_t m = 0;
#pragma unroll
            for (std::uint32_t k = 0; k < 4; ++k) {
                const std::uint32_t b = __float_as_uint(tf32_rna(v[j][k] * sc[j])) & 0x7FFFFFFFu;
                if (f[j] + k < F && b < 0x7F800000u) m = max(m, b);
            }
            if (m) atomicMax(&smax[f[j] / W], m);
        }
    }
    __syncthreads();
    for (std::uint32_t s = threadIdx.x; s < slices; s += blockDim.x)
        if (smax[s]) atomicMax(&partial[(blockIdx.x % kPackSliceMaxRows) * slices + s], smax[s]);
}

__global__ void __launch_bounds__(kThreads) hub_scale_kernel(const std::uint32_t* __restrict__ partial,
                                                            std::uint32_t blocks, std::uint32_t slices,
                                                            float* __restrict__ up, float* __restrict__ down) {
    __shared__ std::uint32_t wmax[kThreads / kWave];
    const std::uint32_t s = blockIdx.x;
    std::uint32_t m = 0;
    for (std::uint32_t b = threadIdx.x; b < blocks; b += blockDim.x)
        m = max(m, partial[static_cast<std::uint64_t>(b) * slices + s]);
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1)
        m = max(m, static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(m), d, kWave)));
    if (__lane_id() == 0) wmax[threadIdx.x / kWave] = m;
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (std::uint32_t w = 1; w < kThreads / kWave; ++w) m = max(m, wmax[w]);
    const int e = m == 0 ? 0 : max(0, min(126, 15 - (static_cast<int>(m >> 23) - 127)));
    up[s] = __uint_as_float(static_cast<std::uint32_t>(127 + e) << 23);
    down[s] = __uint_as_float(static_cast<std::uint32_t>(127 - e) << 23);
}

// As hub_rows_split_kernel over 2^e-scaled values, with half records where
// exact (above).  Thread (pair of column blocks, feature f), W = 32 or 64
// features a slice: the lanes of one slice agree through a ballot, so that
// both column blocks of a binary step hold one form.
__global__ void __launch_bounds__(kThreads) hub_rows_half_kernel(const float* __restrict__ X, std::uint32_t F,
                                     const std::uint32_t* __restrict__ order, std::uint32_t hubCols,
                                     std::uint32_t hubRows, std::uint32_t ldh, const float* __restrict__ colScale,
                                     const float* __restrict__ up, std::uint32_t W, std::uint16_t* __restrict__ Xs,
                                     unsigned char* __restrict__ flags) {
    constexpr std::uint32_t kC = 2 * kTile;
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::uint32_t pr = static_cast<std::uint32_t>(i / ldh), f = static_cast<std::uint32_t>(i % ldh);
    if (pr >= hubRows / kC) return;  // whole waves: ldh is a multiple of 64
    std::uint32_t src[kC];
#pragma unroll
    for (std::uint32_t k = 0; k < kC; ++k) src[k] = order[min(pr * kC + k, hubCols > 0 ? hubCols - 1 : 0u)];
    const std::uint32_t fc = min(f, F > 0 ? F - 1 : 0u);
    float t[kC];
#pragma unroll
    for (std::uint32_t k = 0; k < kC; ++k) t[k] = X[static_cast<std::uint64_t>(src[k]) * F + fc];
    if (colScale) {
#pragma unroll
        for (std::uint32_t k = 0; k < kC; ++k) t[k] *= colScale[src[k]];
    }
    const float sc = up[f / W];
    bool exact = true;
    std::uint32_t h[kC / 2];  // fp16 pairs
#pragma unroll
    for (std::uint32_t k = 0; k < kC; ++k) {
        const bool live = f < F && pr * kC + k < hubCols;
        t[k] = live ? tf32_rna(t[k]) * sc : 0.0f;
        const _Float16 hk = static_cast<_Float16>(t[k]);
        const std::uint32_t hb = __builtin_bit_cast(std::uint16_t, hk);
        h[k / 2] = k % 2 ? h[k / 2] | hb << 16 : hb;
        exact &= __builtin_isnan(t[k]) || __float_as_uint(static_cast<float>(hk)) == __float_as_uint(t[k]);
    }
    // the slice's lanes: all 64 (W = 64) or this lane's half-wave (W = 32)
    const std::uint64_t bad = __ballot(!exact);
    const unsigned lane = __lane_id();
    const bool half = W >= kWave ? bad == 0 : ((bad >> (lane & 32u)) & 0xFFFFFFFFull) == 0;
    // a pair past the hub columns (the zero step's) is zero in both forms:
    // the bf16 layout's 64 bytes per feature cover the fp16 one
    const bool zeroPair = pr * kC >= hubCols;
#pragma unroll
    for (std::uint32_t q = 0; q < 2; ++q) {
        const std::uint64_t cb = 2ull * pr + q;
        if (half && !zeroPair) {
            // dense: feature j of the slice at 32 j bytes of the slice's region
            vu4* hout = reinterpret_cast<vu4*>(Xs + (cb * ldh + f / W * W) * 32 + (f % W) * 16);
            hout[0] = vu4{h[8 * q], h[8 * q + 1], h[8 * q + 2], h[8 * q + 3]};
            hout[1] = vu4{h[8 * q + 4], h[8 * q + 5], h[8 * q + 6], h[8 * q + 7]};
        } else {
            vu4 hi[2], lo[2];
#pragma unroll
            for (std::uint32_t k = 0; k < kTile; k += 2) {
                std::uint16_t h0, l0, h1, l1;
                bf16_split(t[kTile * q + k], h0, l0);
                bf16_split(t[kTile * q + k + 1], h1, l1);
                hi[k / 8][(k % 8) / 2] = static_cast<std::uint32_t>(h0) | static_cast<std::uint32_t>(h1) << 16;
                lo[k / 8][(k % 8) / 2] = static_cast<std::uint32_t>(l0) | static_cast<std::uint32_t>(l1) << 16;
            }
            vu4* out = reinterpret_cast<vu4*>(Xs + (cb * ldh + f) * 32);
            out[0] = hi[0];
            out[1] = hi[1];
            out[2] = lo[0];
            out[3] = lo[1];
        }
    }
    if (f % W == 0) flags[static_cast<std::uint64_t>(pr) * (ldh / W) + f / W] = half ? 1 : 0;
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int G>
struct SplitOperands {
    vu4 a[G];  // lane group q < 2: ah of k = 8q..8q+7; q >= 2: al of k = 8(q-2)..
    vu4 b[4];  // N tile u, feature f0 + 16u + l%16: q < 2 xh of k-half q, q >= 2 xl of k-half q-2
};

// As hub_tiles_kernel, over split tiles.  Per tile and 16 features, two
// K = 32 MFMAs over k' = (lane group q, element e): A' = [ah | al] (lane
// groups 0-1 ah, 2-3 al, of k = 8(q%2) + e) against B = [xh ; xh], then
// against [xl ; xl]: ah·xh + al·xh, then ah·xl + al·xl.  Every lane reads
// its own 16 bytes of the tile and of Xs: lanes 0-31 the xh and lanes 32-63
// the xl of their k-half, and v_permlane32_swap of that register with a
// copy of itself gives [xh ; xh] in one and [xl ; xl] in the other (lanes
// 32-63 of the first take lanes 0-31 of the second, and the reverse; checked
// on the GPU).  D of N tile u holds rows 4q + v, feature f0 + 16u + (l%16).
template <int G, int NS>
__global__ void __launch_bounds__(kThreads) hub_tiles_split_kernel(TileArgs a) {
    const unsigned lane = __lane_id();
    std::uint32_t unit, slice;
    tile_wave(a, unit, slice);
    if (unit >= a.numUnits) return;
    const std::uint32_t g = a.units[3ull * unit], p0 = a.units[3ull * unit + 1], p1 = a.units[3ull * unit + 2];
    if (p0 >= p1) return;
    const std::uint32_t pslot = a.unitPartial[unit];
    const bool shared = pslot != kNoSlot;
    const std::uint32_t f0 = slice * kSlice;
    const unsigned li = lane & 15u, lq = lane >> 4;
    const std::uint32_t last = p1 - 1;
    int cols[kColRegs];
    load_step_cols(a.stepCol, p0, last, cols);
    // Xs: 16 hi then 16 lo bf16 per (column block, feature); lane group q
    // reads bytes 16q..16q+15 (q < 2: xh of k-half q; q >= 2: xl of k-half q-2)
    const char* xb = reinterpret_cast<const char*>(a.Xh) + (static_cast<std::uint64_t>(f0 + li) * 64 + lq * 16);
    const std::uint64_t cbStride = static_cast<std::uint64_t>(a.ldh) * 64;
    // tile: 256 hi then 256 lo bf16, row-major; this lane's row li, k-half, hi or lo
    const char* ab = reinterpret_cast<const char*>(a.tileVals) + (lq >> 1) * 512 + li * 32 + (lq & 1u) * 16;

    auto load = [&](std::uint32_t p, SplitOperands<G>& o) {
        const std::uint32_t pa = p <= last ? p : a.zeroStep;
        const std::uint32_t col = step_col(cols, min(p, last) - p0);
#pragma unroll
        for (int j = 0; j < G; ++j) o.a[j] = load_global<vu4>(ab + (static_cast<std::uint64_t>(pa) * G + j) * (kTileVals * 4));
        const char* rb = xb + col * cbStride;
#pragma unroll
        for (int u = 0; u < 4; ++u) o.b[u] = load_global<vu4>(rb + u * 16 * 64);
    };
    f32x4 acc[G][4];
#pragma unroll
    for (int j = 0; j < G; ++j)
#pragma unroll
        for (int u = 0; u < 4; ++u) acc[j][u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    auto mma = [&](const SplitOperands<G>& o) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            vu4 bh, bl;  // [xh ; xh] and [xl ; xl]
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const auto sw = __builtin_amdgcn_permlane32_swap(o.b[u][r], o.b[u][r], false, false);
                bh[r] = sw[0];
                bl[r] = sw[1];
            }
#pragma unroll
            for (int j = 0; j < G; ++j) {
                const bf16x8 aj = __builtin_bit_cast(bf16x8, o.a[j]);
                acc[j][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aj, __builtin_bit_cast(bf16x8, bh), acc[j][u], 0, 0, 0);
                acc[j][u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aj, __builtin_bit_cast(bf16x8, bl), acc[j][u], 0, 0, 0);
            }
        }
    };

    SplitOperands<G> ring[NS];
#pragma unroll
    for (int k = 0; k < NS - 1; ++k) {
        load(p0 + k, ring[k]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (std::uint32_t p = p0; p < p1; p += NS) {
#pragma unroll
        for (int k = 0; k < NS; ++k) {
            load(p + k + NS - 1, ring[(k + NS - 1) % NS]);
            __builtin_amdgcn_sched_barrier(0);
            mma(ring[k]);
        }
    }

    // D(4*lq + v, li) of N tile u of row block j: row 16j + 4lq + v of the
    // group, feature f0 + 16u + li.
    if (shared) {
        float* base = a.partials + (static_cast<std::uint64_t>(pslot) * G * kTile + 4 * lq) * a.ldh + f0 + li;
#pragma unroll
        for (int j = 0; j < G; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int u = 0; u < 4; ++u) base[static_cast<std::uint64_t>(16 * j + v) * a.ldh + 16 * u] = acc[j][u][v];
        return;
    }
    vu4 rows[G];
#pragma unroll
    for (int j = 0; j < G; ++j)
        rows[j] = load_global<vu4>(a.rowOrder + static_cast<std::uint64_t>(g) * G * kTile + 16 * j + 4 * lq);
    // one row block at a time: its 16 Y values loaded before any is stored
#pragma unroll
    for (int j = 0; j < G; ++j) {
        float y[4][4];
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const std::uint32_t f = f0 + 16 * u + li;
                const bool live = rows[j][v] != TCC_SWTCF_INVALID_ROW_SLOT && f < a.F;
                y[v][u] = live ? a.Y[static_cast<std::uint64_t>(rows[j][v]) * a.F + f] : 0.0f;
            }
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const std::uint32_t f = f0 + 16 * u + li;
                if (rows[j][v] != TCC_SWTCF_INVALID_ROW_SLOT && f < a.F)
                    a.Y[static_cast<std::uint64_t>(rows[j][v]) * a.F + f] = y[v][u] + acc[j][u][v];
            }
    }
}

// Binary tiles (TCC_TILES_BINARY).  The reference's tensor-core operand is
// the block's bitmap as {0, 1} (src/swtcf_spmm.cu:193-200); here the
// patterns of 32-row tiles (row blocks 2t and 2t+1 of a group) by 32
// columns (a pair of 16-column blocks) are the sparse A operand of
// v_smfmac_f32_32x32x32_f16 or _bf16: two value slots per group of four
// columns, with their positions (binary_encode_kernel; a step whose groups
// hold more entries has a second layer).  Lane l supplies row l%32 of the
// tile, slots 0-3 for columns 8(l/32)..+7 of column block 0 and slots 4-7
// for the same columns of block 1; B lane l holds the 16 columns of block
// l/32 for feature l%32; D lane l register r is row 8(r/4) + 4(l/32) + r%4,
// feature l%32 (all checked on the GPU).  The values come as row and column
// scales.  Xs holds 2^e TF32(colScale[c] * X[c]) (e per slice,
// hub_rows_half_kernel): as fp16 values where that is exact for the
// (column-block pair, slice), one f16 product a tile, else as bf16 halves,
// one product against the high parts and one against the low parts.
// Either way sum_c P[i][c] 2^e TF32(c x) is formed from exact products in
// fp32; the sum is multiplied by 2^-e, and by the row scale when it is
// stored.
//
// Expansion: lane l's value-mask byte of tile t (slot j is 1.0 where bit j
// is set) becomes 8 fp16 or bf16 of 0 or 1.0 through one 16-byte read of a
// 256-entry table in LDS; the positions go to the MFMA as they are stored
// (tiles 2u and 2u+1 in the halves of one register).  The next step's
// lookups run between this step's products (G/2 reads).  Every tile of a
// step is multiplied.
//
// One wave per (unit, slice of 32 NT features).  A unit's steps are taken
// 256 at a time (step columns one per lane in four registers), listed by
// record kind, and multiplied in two passes: the fp16 steps (the lane's
// G/2 mask bytes and G bytes of positions, and 2 NT 16-byte Xs loads, then
// G NT / 2 MFMAs) and then the bf16 steps (4 NT Xs loads, G NT MFMAs).
// Loads run NS - 1 steps ahead in a ring of NS stages (2 for the bf16
// steps, whose stages are twice the registers), as in the valued kernels.
template <int G, int NT>
struct BinaryStage {
    std::uint32_t m[G / 8];   // this lane's G/2 value-mask bytes (byte t: 32-row tile t)
    std::uint32_t ix[G / 4];  // positions: tile t in bits 16(t%2).. of word t/2
    vu4 h[NT][2];             // N tile u: 16 fp16 x (or bf16 xh) of column block l/32, feature f0 + 32u + l%32
    vu4 lo[NT][2];            // the same columns' xl (bf16 records)
};

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x16 __attribute__((ext_vector_type(16)));
typedef std::uint32_t vu8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ vu8 join8(const vu4& a, const vu4& b) {
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// acc += A B on the sparse MFMA; HI selects the upper 16 position bits of ix.
template <bool HALF, int HI>
__device__ __forceinline__ f32x16 smfmac(const vu4& A, const vu8& B, const f32x16& acc, std::uint32_t ix) {
    if constexpr (HALF)
        return __builtin_amdgcn_smfmac_f32_32x32x32_f16(__builtin_bit_cast(f16x8, A), __builtin_bit_cast(f16x16, B), acc,
                                                        static_cast<int>(ix), 0, HI);
    else
        return __builtin_amdgcn_smfmac_f32_32x32x32_bf16(__builtin_bit_cast(bf16x8, A), __builtin_bit_cast(bf16x16, B),
                                                         acc, static_cast<int>(ix), 0, HI);
}

template <int G, int NT, int NS>
__global__ void __launch_bounds__(kThreads) hub_tiles_binary_kernel(TileArgs a) {
    static_assert(G == 8 || G == 16, "binary tiles: G is 8 or 16");
    constexpr int T = G / 2;  // 32-row tiles a step
    // lut[x] = 8 fp16 (0 or 1.0) of the 8 bits of x, low bit first, then
    // lut[256 + x] the same in bf16
    __shared__ vu4 lut[512];
    // each wave's steps of the current stretch: fp16 steps from the front,
    // bf16 steps from the back, as (column-block pair << 8 | step - c0)
    __shared__ std::uint32_t stepList[kThreads / kWave][kMaxUnitSteps];
    for (unsigned e = threadIdx.x; e < 512; e += blockDim.x) {
        const unsigned x = e & 255u, one = e < 256 ? 0x3C00u : 0x3F80u;
        auto pair = [one](unsigned y) { return ((y & 1u) ? one : 0u) | ((y & 2u) ? one << 16 : 0u); };
        lut[e] = vu4{pair(x & 3u), pair((x >> 2) & 3u), pair((x >> 4) & 3u), pair(x >> 6)};
    }
    __syncthreads();
    const char* lutBytes = reinterpret_cast<const char*>(lut);
    const unsigned lane = __lane_id();
    std::uint32_t unit, slice;
    tile_wave(a, unit, slice);
    if (unit >= a.numUnits) return;
    const std::uint32_t g = a.units[3ull * unit], p0 = a.units[3ull * unit + 1], p1 = a.units[3ull * unit + 2];
    if (p0 >= p1) return;
    const std::uint32_t pslot = a.unitPartial[unit];
    const std::uint32_t f0 = slice * (32 * NT);
    const unsigned lj = lane & 31u, lh = lane >> 5;
    // Xs per (column block, slice): bf16 records of 16 hi then 16 lo values
    // per feature (64 bytes), or fp16 records of 16 values per feature (32
    // bytes, the slice's first half); this lane's column block of the pair
    const std::uint64_t cbStride = static_cast<std::uint64_t>(a.ldh) * 64;
    const char* xb = reinterpret_cast<const char*>(a.Xh) + (lh * cbStride + static_cast<std::uint64_t>(f0 + lj) * 64);
    const char* xbh = reinterpret_cast<const char*>(a.Xh) + (lh * cbStride + static_cast<std::uint64_t>(f0) * 64 + lj * 32);
    // sub-step records of 96 G bytes: value masks (G/2 bytes a lane), then positions (G bytes a lane)
    const std::uint32_t* mb = a.tileMasks + lane * (G / 8);
    const std::uint32_t* ib = a.tileMasks + 8 * G + lane * (G / 4);
    std::uint32_t* list = stepList[threadIdx.x / kWave];

    f32x16 acc[T][NT];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int u = 0; u < NT; ++u)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[t][u][r] = 0.0f;

    // One pass of the ring over `count` listed steps (entry i at base[i]),
    // all fp16 (HALF) or all bf16 records: the two kinds of product stay in
    // separate loops (one loop holding both took the accumulators out of
    // place, 230 AGPRs and one wave per SIMD).
    auto run = [&](auto halfTag, const int (&ents)[kColRegs], std::uint32_t count, std::uint32_t c0) {
        constexpr bool HALF = decltype(halfTag)::value;
        constexpr int K = HALF ? NS : 2;  // ring stages
        const char* lb = lutBytes + (HALF ? 0 : 4096);
        // Listed step i (i >= count: the zero step, multiplying zeros by
        // zeros; B read from a real step's column would turn an inf there
        // into NaN in every row).
        auto load = [&](std::uint32_t i, BinaryStage<G, NT>& o) {
            const bool live = i < count;
            const std::uint32_t e = step_col(ents, live ? i : 0);
            const std::uint32_t pa = live ? c0 + (e & 0xFFu) : a.zeroStep;
            const std::uint32_t col = live ? e >> 8 : a.zeroCol;
            const std::uint64_t rec = static_cast<std::uint64_t>(pa) * (24 * G);
            if constexpr (G == 16) {
                const vu2 w = load_global<vu2>(mb + rec);
                o.m[0] = w.x;
                o.m[1] = w.y;
                const vu4 q = load_global<vu4>(ib + rec);
                o.ix[0] = q.x;
                o.ix[1] = q.y;
                o.ix[2] = q.z;
                o.ix[3] = q.w;
            } else {
                o.m[0] = load_global<std::uint32_t>(mb + rec);
                const vu2 q = load_global<vu2>(ib + rec);
                o.ix[0] = q.x;
                o.ix[1] = q.y;
            }
            // unconditional loads (the zero step reads the pair of zeros):
            // a load under a branch split the ring into blocks that waited
            // for each step's loads before its products
            const char* rb = (HALF ? xbh : xb) + static_cast<std::uint64_t>(col) * 2 * cbStride;
#pragma unroll
            for (int u = 0; u < NT; ++u) {
                const char* ru = rb + u * 32 * (HALF ? 32 : 64);
                o.h[u][0] = load_global<vu4>(ru);
                o.h[u][1] = load_global<vu4>(ru + 16);
                if constexpr (!HALF) {
                    o.lo[u][0] = load_global<vu4>(ru + 32);
                    o.lo[u][1] = load_global<vu4>(ru + 48);
                }
            }
        };
        // every tile's lookups of one step: byte addresses 16 * mask byte
        auto expand = [&](const BinaryStage<G, NT>& o, vu4 (&A)[T]) {
#pragma unroll
            for (int w = 0; w < G / 8; ++w) {
#pragma unroll
                for (int q = 0; q < 4 && 4 * w + q < T; ++q) {
                    const std::uint32_t b = q == 0 ? (o.m[w] & 0xFFu) : __builtin_amdgcn_ubfe(o.m[w], 8 * q, 8);
                    A[4 * w + q] = *reinterpret_cast<const vu4*>(lb + (b << 4));
                }
            }
        };
        auto mma = [&](const vu4 (&A)[T], const BinaryStage<G, NT>& o) {
#pragma unroll
            for (int t = 0; t < T; ++t) {
#pragma unroll
                for (int u = 0; u < NT; ++u) {
                    const std::uint32_t ix = o.ix[t / 2];
                    const vu8 bh = join8(o.h[u][0], o.h[u][1]);
                    if (t % 2) acc[t][u] = smfmac<HALF, 1>(A[t], bh, acc[t][u], ix);
                    else acc[t][u] = smfmac<HALF, 0>(A[t], bh, acc[t][u], ix);
                    if constexpr (!HALF) {
                        const vu8 bl = join8(o.lo[u][0], o.lo[u][1]);
                        if (t % 2) acc[t][u] = smfmac<HALF, 1>(A[t], bl, acc[t][u], ix);
                        else acc[t][u] = smfmac<HALF, 0>(A[t], bl, acc[t][u], ix);
                    }
                }
            }
        };

        BinaryStage<G, NT> ring[K];
#pragma unroll
        for (int k = 0; k < K - 1; ++k) {
            load(k, ring[k]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // A step's operands are expanded while the previous step's products
        // run (the lookups' latency hides behind the MFMAs).
        vu4 A[T];
        expand(ring[0], A);
        for (std::uint32_t i = 0; i < count; i += K) {
#pragma unroll
            for (int k = 0; k < K; ++k) {
                load(i + k + K - 1, ring[(k + K - 1) % K]);
                __builtin_amdgcn_sched_barrier(0);
                mma(A, ring[k]);
                expand(ring[(k + 1) % K], A);
                // one MFMA, then a lookup and VALU instructions of the next
                // step's expansion, and so on: the next step's lookups run
                // between this step's products
                constexpr int kMfma = (HALF ? 1 : 2) * T * NT;
#pragma unroll
                for (int j = 0; j < kMfma; ++j) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x002, HALF ? 2 : 1, 0);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };

    for (std::uint32_t c0 = p0; c0 < p1; c0 += kMaxUnitSteps) {
        const std::uint32_t last = min(c0 + kMaxUnitSteps, p1) - 1;
        int cols[kColRegs];
        load_step_cols_flagged(a.stepCol, c0, last, cols, a.halfFlags, a.slices, slice);
        // the stretch's steps listed by kind, in step order within each
        std::uint32_t nh = 0, nf = 0;
#pragma unroll
        for (int k = 0; k < kColRegs; ++k) {
            const std::uint32_t q = 64u * k + lane;
            const bool valid = c0 + q <= last;
            const std::uint32_t cw = static_cast<std::uint32_t>(cols[k]);
            const bool isHalf = valid && (cw >> 31) != 0, isFull = valid && (cw >> 31) == 0;
            const std::uint64_t bh = __ballot(isHalf), bf = __ballot(isFull);
            const std::uint32_t entry = (cw & 0x7FFFFFFFu) << 8 | q;
            if (isHalf) list[nh + __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(bh >> 32),
                                                           __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(bh), 0u))] = entry;
            if (isFull) list[kMaxUnitSteps - 1 - (nf + __builtin_amdgcn_mbcnt_hi(static_cast<std::uint32_t>(bf >> 32),
                                                           __builtin_amdgcn_mbcnt_lo(static_cast<std::uint32_t>(bf), 0u)))] = entry;
            nh += static_cast<std::uint32_t>(__popcll(bh));
            nf += static_cast<std::uint32_t>(__popcll(bf));
        }
        __builtin_amdgcn_wave_barrier();
        // the lists back in registers, entry i in lane i % 64 of register i / 64
        int ents[kColRegs];
        if (nh) {
#pragma unroll
            for (int k = 0; k < kColRegs; ++k) ents[k] = static_cast<int>(list[64 * k + lane]);
            run(std::true_type{}, ents, nh, c0);
        }
        if (nf) {
#pragma unroll
            for (int k = 0; k < kColRegs; ++k)
                ents[k] = static_cast<int>(list[min(kMaxUnitSteps - nf + 64 * k + lane, kMaxUnitSteps - 1)]);
            run(std::false_type{}, ents, nf, c0);
        }
        __builtin_amdgcn_wave_barrier();
    }
    // the slice's scale undone (an exact power of two)
    if (a.sliceDown) {
        const float down = a.sliceDown[slice];
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int u = 0; u < NT; ++u) acc[t][u] *= down;
    }

    // D register r of tile t, N tile u: row 32t + 8(r/4) + 4lh + r%4 of the
    // group, feature f0 + 32u + lj.
    if (pslot != kNoSlot) {
        float* base = a.partials + (static_cast<std::uint64_t>(pslot) * G * kTile + 4 * lh) * a.ldh + f0 + lj;
#pragma unroll
        for (int t = 0; t < T; ++t)
#pragma unroll
            for (int r = 0; r < 16; ++r)
#pragma unroll
                for (int u = 0; u < NT; ++u)
                    base[static_cast<std::uint64_t>(32 * t + 8 * (r / 4) + r % 4) * a.ldh + 32 * u] = acc[t][u][r];
        return;
    }
    // four rows at a time (one 16-byte load of their order and scales), their
    // Y values loaded before any is stored
    const std::uint64_t gs = static_cast<std::uint64_t>(g) * G * kTile + 4 * lh;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int rq = 0; rq < 4; ++rq) {
            const std::uint64_t s4 = gs + 32 * t + 8 * rq;
            const vu4 rows = load_global<vu4>(a.rowOrder + s4);
            const f32x4 rsc = a.rowScale ? load_global<vf4>(a.rowScale + s4) : f32x4{1.0f, 1.0f, 1.0f, 1.0f};
            float y[4][NT];
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int u = 0; u < NT; ++u) {
                    const std::uint32_t f = f0 + 32 * u + lj;
                    const bool live = rows[v] != TCC_SWTCF_INVALID_ROW_SLOT && f < a.F && !a.storeY;
                    y[v][u] = live ? a.Y[static_cast<std::uint64_t>(rows[v]) * a.F + f] : 0.0f;
                }
#pragma unroll
            for (int v = 0; v < 4; ++v)
#pragma unroll
                for (int u = 0; u < NT; ++u) {
                    const std::uint32_t f = f0 + 32 * u + lj;
                    if (rows[v] != TCC_SWTCF_INVALID_ROW_SLOT && f < a.F)
                        a.Y[static_cast<std::uint64_t>(rows[v]) * a.F + f] = y[v][u] + rsc[v] * acc[t][u][4 * rq + v];
                }
        }
}

// Y rows of a shared group += the sum of its units' partials (times the
// row scales of binary tiles), one workgroup per (shared group, 64-feature
// slice, row block j of the group): thread q sums row 16j + q/16, features
// 4(q%16)..+3 of the slice over the group's units in unit order (their
// slots are consecutive), sixteen loads in flight (the core's first groups
// have dozens of units).
__global__ void __launch_bounds__(kThreads) hub_reduce_kernel(TileArgs a, std::uint32_t G) {
    const std::uint32_t rslices = a.ldh / kSlice;
    const std::uint32_t per = rslices * G;
    const std::uint32_t sg = blockIdx.x / per, rest = blockIdx.x - sg * per;
    const std::uint32_t slice = rest / G, j = rest - slice * G;
    const std::uint32_t g = a.sharedGroups[3ull * sg], slot0 = a.sharedGroups[3ull * sg + 1];
    const std::uint32_t nu = a.sharedGroups[3ull * sg + 2];
    const std::uint32_t f = slice * kSlice + 4 * (threadIdx.x % 16);
    const unsigned r = 16 * j + threadIdx.x / 16;
    const std::uint64_t stride = static_cast<std::uint64_t>(G) * kTile * a.ldh;  // one unit's partials
    const float* p = a.partials + (static_cast<std::uint64_t>(slot0) * G * kTile + r) * a.ldh + f;
    constexpr std::uint32_t kIn = 16;
    f32x4 s[kIn];
#pragma unroll
    for (std::uint32_t i = 0; i < kIn; ++i) s[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    std::uint32_t k = 0;
    for (; k + kIn <= nu; k += kIn)
#pragma unroll
        for (std::uint32_t i = 0; i < kIn; ++i) s[i] += load_global<vf4>(p + (k + i) * stride);
    for (; k < nu; ++k) s[0] += load_global<vf4>(p + k * stride);
#pragma unroll
    for (std::uint32_t i = 1; i < kIn; ++i) s[0] += s[i];
    const std::uint64_t slotRow = static_cast<std::uint64_t>(g) * G * kTile + r;
    const std::uint32_t orow = a.rowOrder[slotRow];
    if (orow == TCC_SWTCF_INVALID_ROW_SLOT) return;
    if (a.rowScale) s[0] *= a.rowScale[slotRow];
    const bool vec = a.F % 4 == 0 && (reinterpret_cast<std::uintptr_t>(a.Y) & 15u) == 0;
    add_quad(a.Y + static_cast<std::uint64_t>(orow) * a.F, f, a.F, vec, s[0], a.storeY != 0);
}

// With storeY: zero the Y rows no unit writes, those of the groups without
// steps and the padding rows numRows..outRows-1: wave w of the grid takes row
// slot w (slots of rowOrder first, then the padding rows), a row of F floats
// in coalesced stores.
__global__ void __launch_bounds__(kThreads) hub_zero_rows_kernel(TileArgs a, std::uint32_t G, std::uint32_t numSlots,
                                                                std::uint32_t numRows, std::uint32_t outRows) {
    const std::uint32_t w = (blockIdx.x * blockDim.x + threadIdx.x) / kWave;
    std::uint32_t row;
    if (w < numSlots) {
        const std::uint32_t g = w / (G * kTile);
        if (a.groupStepOffset[g + 1] > a.groupStepOffset[g]) return;  // its units write its rows
        row = a.rowOrder[w];
        if (row == TCC_SWTCF_INVALID_ROW_SLOT) return;
    } else if (w < numSlots + (outRows - numRows)) {
        row = numRows + (w - numSlots);
    } else {
        return;
    }
    float* y = a.Y + static_cast<std::uint64_t>(row) * a.F;
    for (std::uint32_t f = __lane_id(); f < a.F; f += kWave) y[f] = 0.0f;
}

inline std::uint32_t hub_ldh(std::uint32_t F) { return (F + kSlice - 1) / kSlice * kSlice; }

// rows of Xh: the hub columns rounded up to whole column blocks; for
// binary tiles to pairs of them, plus one pair of zeros (the zero step's
// columns: every load of the ring's tail reads a real address)
inline std::uint32_t hub_rows(const tcc_hub_tiles* T) {
    if (T->tile_format == TCC_TILES_BINARY) return (T->hub_cols + 2 * kTile - 1) / (2 * kTile) * (2 * kTile) + 2 * kTile;
    return (T->hub_cols + kTile - 1) / kTile * kTile;
}

// Two steps in flight (three stages) for the small groups; the larger
// groups keep their 4 G accumulator tiles and two stages within two or
// more waves per SIMD (the accumulators sit in arch VGPRs: the library
// builds this file with -amdgpu-mfma-vgpr-form, and the split kernel takes
// 244 registers at G = 8 where the AGPR form took 392).
template <int G>
hipError_t launch_tiles(const TileArgs& a, bool split, hipStream_t st) {
    constexpr int NS = G <= 2 ? 3 : 2;
    // split tiles: two stages (a third measured slower at G = 4, equal at G = 8)
    if (split)
        hipLaunchKernelGGL((hub_tiles_split_kernel<G, 2>), dim3(kXcds * tiles_blocks_per_xcd(a.numUnits, a.slices)),
                           dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL((hub_tiles_kernel<G, NS>), dim3(kXcds * tiles_blocks_per_xcd(a.numUnits, a.slices)),
                           dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

// Binary tiles: G/2 32-row tiles by NT 32-feature N tiles of 16
// accumulators (128 registers): one N tile at G = 16 (32 features a wave),
// two at G = 8 (64 features a wave).
constexpr int binary_nt(std::uint32_t G) { return G == 16 ? 1 : 2; }
// Loads of fp16 steps run three steps ahead (bf16 steps, whose stages hold
// twice the registers, one step ahead): 242 registers at G = 16, two waves
// per SIMD.
constexpr int kBinaryStages = 4;

hipError_t launch_binary(const TileArgs& a, std::uint32_t G, hipStream_t st) {
    const dim3 grid(kXcds * tiles_blocks_per_xcd(a.numUnits, a.slices));
    if (G == 16)
        hipLaunchKernelGGL((hub_tiles_binary_kernel<16, binary_nt(16), kBinaryStages>), grid, dim3(kThreads), 0, st, a);
    else
        hipLaunchKernelGGL((hub_tiles_binary_kernel<8, binary_nt(8), kBinaryStages>), grid, dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

struct HybridParams {
    const std::uint32_t* row;
    const std::uint32_t* col;
    const float* val;
    std::uint32_t nnz;
    std::uint32_t numRows;
    std::uint32_t numCols;
    std::uint32_t minStepNnz;
    std::uint32_t minTileNnz;
    std::uint32_t G;
    std::uint32_t unitSteps;
    std::uint32_t format;
    std::uint32_t phases;
    const float* rowScale;  // binary tiles
    const float* colScale;
};

// The hub tiles and the remainder's (phased) BCSR of a device COO; see
// tcc_coo_to_hybrid and tcc_coo_to_hybrid_scaled.
int build_hybrid(const HybridParams& P, tcc_hybrid* out, void* stream) {
    const hipStream_t st = as_stream(stream);
    const bool binary = P.format == TCC_TILES_BINARY;
    std::memset(out, 0, sizeof(*out));
    const std::uint32_t E = P.nnz, numRows = P.numRows, numCols = P.numCols, G = P.G;
    const std::uint32_t RB = (numRows + kTile - 1) / kTile;
    const std::uint32_t NG = (RB + G - 1) / G;
    const std::uint32_t rowSlots = NG * G * kTile;
    // binary steps pair 16-column blocks: the block count rounded up to even
    const std::uint32_t CB = (numCols + kTile - 1) / kTile + (binary ? ((numCols + kTile - 1) / kTile) % 2 : 0);
    const std::uint32_t stepTiles = binary ? 2 * G : G, colSteps = binary ? CB / 2 : CB;
    const std::uint64_t En = std::max<std::uint32_t>(E, 1);
    const std::uint64_t Vn = std::max<std::uint64_t>({En, rowSlots, numCols});
    const unsigned tileBits = std::max(1u, rank_bits(static_cast<std::uint64_t>(NG) * CB * G));
    TCC_REQUIRE(tileBits + 8 <= 64, TCC_ERR_UNSUPPORTED, "hybrid: tile key exceeds 64 bits");
    const std::uint64_t tempElems = std::max({radix_temp_elems(Vn), scan_temp_elems(En + 1),
                                              scan_temp_elems(static_cast<std::uint64_t>(NG) + 1)});

    std::uint64_t *keysA, *keysB;
    std::uint32_t *permA, *permB, *flags, *pos, *tileStart, *dense, *stepHead, *stepPos, *slot, *restFlag, *restPos,
        *rowDeg, *colDeg, *rowRank, *colRank, *rowOrder, *colOrder, *groupSteps, *unitCount, *temp, *small, *restRow,
        *restCol;
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
        stepHead = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        stepPos = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        slot = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        restFlag = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        restPos = reinterpret_cast<std::uint32_t*>(take(4 * (En + 1)));
        rowDeg = reinterpret_cast<std::uint32_t*>(take(4 * (numRows + 1)));
        colDeg = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        rowRank = reinterpret_cast<std::uint32_t*>(take(4 * (numRows + 1)));
        colRank = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        rowOrder = reinterpret_cast<std::uint32_t*>(take(4ull * rowSlots));
        colOrder = reinterpret_cast<std::uint32_t*>(take(4 * (numCols + 1)));
        groupSteps = reinterpret_cast<std::uint32_t*>(take(4 * (NG + 1)));
        unitCount = reinterpret_cast<std::uint32_t*>(take(4 * (NG + 1)));
        restRow = reinterpret_cast<std::uint32_t*>(take(4 * En));
        restCol = reinterpret_cast<std::uint32_t*>(take(4 * En));
        restVal = reinterpret_cast<float*>(take(4 * En));
        temp = reinterpret_cast<std::uint32_t*>(take(4 * tempElems));
        // [0]=err [1]=tiles [2]=steps [3]=rest [4]=units [5]=hubBlocks [6]=dense tiles [7]=sub-steps
        small = reinterpret_cast<std::uint32_t*>(take(256));
        return off;
    };
    const std::size_t scratchBytes = carve(nullptr);
    DevBuf<char> scratch;
    TCC_HIP_CHECK(hipMalloc(&scratch.p, scratchBytes));
    carve(scratch.p);

    TCC_HIP_CHECK(fill<std::uint32_t>(small, 64, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(rowDeg, numRows, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(colDeg, numCols, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(groupSteps, NG + 1, 0u, st));
    // dense[] and stepHead[] are scanned over E entries; only the first
    // (tile count) are set below
    TCC_HIP_CHECK(fill<std::uint32_t>(dense, En, 0u, st));
    TCC_HIP_CHECK(fill<std::uint32_t>(stepHead, En, 0u, st));
    TCC_HIP_CHECK(degree_histogram(P.row, E, numRows, rowDeg, small, st));
    TCC_HIP_CHECK(degree_histogram(P.col, E, numCols, colDeg, small, st));
    std::uint32_t hostSmall[8] = {};
    TCC_HIP_CHECK(hipMemcpyAsync(hostSmall, small, sizeof(hostSmall), hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    TCC_REQUIRE(hostSmall[0] == 0, TCC_ERR_INVALID_ARGUMENT, "COO index out of range");
    TCC_HIP_CHECK(degree_ranks(rowDeg, numRows, rowSlots, rowRank, rowOrder, keysA, keysB, temp, st));
    TCC_HIP_CHECK(degree_ranks(colDeg, numCols, numCols, colRank, colOrder, keysA, keysB, temp, st));

    std::uint64_t* sorted = keysA;
    std::uint32_t* perm = permA;
    if (E > 0) {
        hipLaunchKernelGGL(tile_keys_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, P.row, P.col, E,
                           rowRank, colRank, CB, G, keysA, permA);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(radix_sort_pairs(keysA, keysB, permA, permB, E, tileBits + 8, temp, &sorted, &perm, st));
        hipLaunchKernelGGL(tile_heads_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, E, flags, small);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(flags, pos, E, small + 1, temp, st));
        hipLaunchKernelGGL(tile_start_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, flags, pos, E,
                           tileStart);
        hipLaunchKernelGGL(dense_tiles_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, tileStart,
                           small + 1, E, P.minTileNnz, P.minStepNnz, colSteps, stepTiles, dense, small + 6, small + 5);
        hipLaunchKernelGGL(step_heads_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, tileStart,
                           small + 1, dense, stepTiles, colSteps, stepHead, groupSteps);
        TCC_LAUNCH_CHECK();
        // step positions over the E-sized head array (zero past the tile count)
        TCC_HIP_CHECK(exclusive_scan(stepHead, stepPos, E, small + 2, temp, st));
        hipLaunchKernelGGL(rest_flags_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, flags, pos, dense, E,
                           restFlag);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(restFlag, restPos, E, small + 3, temp, st));
    }
    if (!binary) {
        hipLaunchKernelGGL(units_per_group_kernel, dim3(grid_for(NG, kThreads)), dim3(kThreads), 0, st, groupSteps, NG,
                           P.unitSteps, unitCount);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(unitCount, unitCount, NG, small + 4, temp, st));
    }
    TCC_HIP_CHECK(hipMemcpyAsync(hostSmall, small, sizeof(hostSmall), hipMemcpyDeviceToHost, st));
    TCC_HIP_CHECK(hipStreamSynchronize(st));
    TCC_REQUIRE(hostSmall[0] == 0, TCC_ERR_INVALID_ARGUMENT,
                hostSmall[0] == 2 ? "duplicate (row, col) entries in the COO input" : "COO index out of range");
    const std::uint32_t NS = E > 0 ? hostSmall[2] : 0;
    const std::uint32_t NR = E > 0 ? hostSmall[3] : 0;
    const std::uint32_t ND = E > 0 ? hostSmall[6] : 0;
    const std::uint32_t hubCols = std::min(hostSmall[5] * (binary ? 2 * kTile : kTile), numCols);

    // Binary tiles: the steps' raw bits, their layers (a second one where a
    // nibble holds more than two entries) and the sub-steps the units cut.
    std::uint32_t NSS = NS;  // sub-steps
    DevBuf<char> binScratch;
    std::uint32_t *raw = nullptr, *stepColTmp = nullptr, *subPos = nullptr, *subOffset = nullptr;
    if (binary) {
        const std::uint64_t NS1 = static_cast<std::uint64_t>(NS) + 1;
        std::uint32_t *stepOffset, *layers, *groupSub;
        auto carveBin = [&](char* base) {
            std::size_t off = 0;
            auto take = [&](std::size_t bytes) {
                char* p = base ? base + off : nullptr;
                off += align_up(bytes);
                return reinterpret_cast<std::uint32_t*>(p);
            };
            raw = take(64ull * G * NS1);
            stepColTmp = take(4 * NS1);
            stepOffset = take(4ull * (NG + 1));
            layers = take(4 * NS1);
            subPos = take(4 * NS1);
            subOffset = take(4ull * (NG + 1));
            groupSub = take(4ull * (NG + 1));
            return off;
        };
        TCC_HIP_CHECK(hipMalloc(&binScratch.p, carveBin(nullptr)));
        carveBin(binScratch.p);
        TCC_HIP_CHECK(fill<std::uint32_t>(raw, 16ull * G * NS1, 0u, st));
        if (E > 0) {
            hipLaunchKernelGGL(tile_slots_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, tileStart,
                               small + 1, dense, stepHead, stepPos, stepTiles, colSteps, slot, stepColTmp);
            hipLaunchKernelGGL(place_entries_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, perm,
                               E, flags, pos, dense, slot, restPos, P.row, P.col, P.val, nullptr, P.format, G, raw,
                               restRow, restCol, P.val ? restVal : nullptr);
            TCC_LAUNCH_CHECK();
        }
        TCC_HIP_CHECK(exclusive_scan(groupSteps, stepOffset, NG, stepOffset + NG, temp, st));
        if (NS > 0) {
            hipLaunchKernelGGL(binary_layers_kernel, dim3(grid_for(static_cast<std::uint64_t>(NS) * kWave, kThreads)),
                               dim3(kThreads), 0, st, raw, NS, G, layers);
            TCC_LAUNCH_CHECK();
        }
        TCC_HIP_CHECK(exclusive_scan(layers, subPos, NS, subPos + NS, temp, st));
        hipLaunchKernelGGL(sub_offsets_kernel, dim3(grid_for(NG + 1, kThreads)), dim3(kThreads), 0, st, stepOffset,
                           subPos, NG, subOffset, groupSub);
        hipLaunchKernelGGL(units_per_group_kernel, dim3(grid_for(NG, kThreads)), dim3(kThreads), 0, st, groupSub, NG,
                           P.unitSteps, unitCount);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(unitCount, unitCount, NG, small + 4, temp, st));
        TCC_HIP_CHECK(hipMemcpyAsync(small + 7, subPos + NS, 4, hipMemcpyDeviceToDevice, st));
        TCC_HIP_CHECK(hipMemcpyAsync(hostSmall, small, sizeof(hostSmall), hipMemcpyDeviceToHost, st));
        TCC_HIP_CHECK(hipStreamSynchronize(st));
        NSS = hostSmall[7];
    }
    const std::uint32_t NU = hostSmall[4];

    // tiles part: rowOrder[rowSlots] hubColOrder[hubCols] groupStepOffset[NG+1] unitFirst[NG+1] stepCol[NS]
    // units[3 NU] unitOrder[NU] unitPartial[NU] sharedGroups[3 NG] then the format's tiles (one more step, of
    // zeros, that the kernels' ring tail reads): tileVals[256 G (NS+1)], or tileMasks[8 G (NS+1)] and the
    // scales
    const std::uint64_t NSn = std::max<std::uint32_t>(NSS, 1);
    const std::uint64_t NUn = std::max<std::uint32_t>(NU, 1);
    const std::uint32_t paddedRows = (numRows + 7) / 8 * 8;
    std::size_t tilesBytes = align_up(4ull * rowSlots) + align_up(4ull * std::max(hubCols, 1u)) +
                             align_up(4ull * (NG + 1)) + align_up(4ull * (NG + 1)) + align_up(4 * NSn) +
                             align_up(12 * NUn) + align_up(4 * NUn) + align_up(4 * NUn) + align_up(12ull * NG);
    if (binary) {
        tilesBytes += align_up(96ull * G * (NSS + 1));
        if (P.rowScale) tilesBytes += align_up(4ull * rowSlots) + align_up(4ull * paddedRows);
        if (P.colScale) tilesBytes += align_up(4ull * numCols);
    } else {
        tilesBytes += align_up(4ull * kTileVals * G * (NS + 1));
    }
    char* o = nullptr;
    TCC_HIP_CHECK(hipMalloc(&o, tilesBytes));
    char* q = o;
    auto takeOut = [&](std::size_t bytes) {
        char* p = q;
        q += align_up(bytes);
        return p;
    };
    auto* oRowOrder = reinterpret_cast<std::uint32_t*>(takeOut(4ull * rowSlots));
    auto* oHubCols = reinterpret_cast<std::uint32_t*>(takeOut(4ull * std::max(hubCols, 1u)));
    auto* oGroupStepOffset = reinterpret_cast<std::uint32_t*>(takeOut(4ull * (NG + 1)));
    auto* oUnitFirst = reinterpret_cast<std::uint32_t*>(takeOut(4ull * (NG + 1)));
    auto* oStepCol = reinterpret_cast<std::uint32_t*>(takeOut(4 * NSn));
    auto* oUnits = reinterpret_cast<std::uint32_t*>(takeOut(12 * NUn));
    auto* oUnitOrder = reinterpret_cast<std::uint32_t*>(takeOut(4 * NUn));
    auto* oUnitPartial = reinterpret_cast<std::uint32_t*>(takeOut(4 * NUn));
    auto* oSharedGroups = reinterpret_cast<std::uint32_t*>(takeOut(12ull * NG));
    float* oTileVals = nullptr;
    std::uint32_t* oTileMasks = nullptr;
    float *oRowScale = nullptr, *oRestRowScale = nullptr, *oColScale = nullptr;
    if (binary) {
        oTileMasks = reinterpret_cast<std::uint32_t*>(takeOut(96ull * G * (NSS + 1)));
        if (P.rowScale) {
            oRowScale = reinterpret_cast<float*>(takeOut(4ull * rowSlots));
            oRestRowScale = reinterpret_cast<float*>(takeOut(4ull * paddedRows));
        }
        if (P.colScale) oColScale = reinterpret_cast<float*>(takeOut(4ull * numCols));
    } else {
        oTileVals = reinterpret_cast<float*>(takeOut(4ull * kTileVals * G * (NS + 1)));
    }
    auto fail = [&](int rc) {
        (void)hipFree(o);
        return rc;
    };
    bool ok = hipMemcpyAsync(oRowOrder, rowOrder, 4ull * rowSlots, hipMemcpyDeviceToDevice, st) == hipSuccess &&
              (!hubCols || hipMemcpyAsync(oHubCols, colOrder, 4ull * hubCols, hipMemcpyDeviceToDevice, st) == hipSuccess) &&
              (binary ? hipMemcpyAsync(oGroupStepOffset, subOffset, 4ull * (NG + 1), hipMemcpyDeviceToDevice, st)
                      : exclusive_scan(groupSteps, oGroupStepOffset, NG, oGroupStepOffset + NG, temp, st)) == hipSuccess &&
              hipMemcpyAsync(oUnitFirst, unitCount, 4ull * NG, hipMemcpyDeviceToDevice, st) == hipSuccess &&
              hipMemcpyAsync(oUnitFirst + NG, small + 4, 4, hipMemcpyDeviceToDevice, st) == hipSuccess;
    if (binary) {
        ok = ok && fill<std::uint32_t>(oTileMasks, 24ull * G * (NSS + 1), 0u, st) == hipSuccess;
        if (ok && NS > 0)
            hipLaunchKernelGGL(binary_encode_kernel, dim3(grid_for(static_cast<std::uint64_t>(NS) * kWave, kThreads)),
                               dim3(kThreads), 0, st, raw, NS, G, subPos, stepColTmp, oTileMasks, oStepCol);
        if (ok && P.rowScale) {
            hipLaunchKernelGGL(ordered_scale_kernel, dim3(grid_for(rowSlots, kThreads)), dim3(kThreads), 0, st,
                               oRowOrder, rowSlots, P.rowScale, oRowScale);
            hipLaunchKernelGGL(padded_copy_kernel, dim3(grid_for(paddedRows, kThreads)), dim3(kThreads), 0, st,
                               P.rowScale, numRows, paddedRows, oRestRowScale);
        }
        if (ok && P.colScale)
            hipLaunchKernelGGL(padded_copy_kernel, dim3(grid_for(numCols, kThreads)), dim3(kThreads), 0, st,
                               P.colScale, numCols, numCols, oColScale);
    } else {
        ok = ok && fill<float>(oTileVals, kTileVals * G * (NS + 1ull), 0.0f, st) == hipSuccess;
    }
    if (!ok || hipGetLastError() != hipSuccess) {
        set_last_error("HIP error while initialising the hub tiles");
        return fail(TCC_ERR_HIP);
    }
    if (E > 0 && !binary) {
        hipLaunchKernelGGL(tile_slots_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, tileStart,
                           small + 1, dense, stepHead, stepPos, stepTiles, colSteps, slot, oStepCol);
        hipLaunchKernelGGL(place_entries_kernel, dim3(grid_for(E, kThreads)), dim3(kThreads), 0, st, sorted, perm, E,
                           flags, pos, dense, slot, restPos, P.row, P.col, P.val, oTileVals, P.format, G, oTileMasks,
                           restRow, restCol, P.val ? restVal : nullptr);
    }
    hipLaunchKernelGGL(group_units_kernel, dim3(grid_for(NG, kThreads)), dim3(kThreads), 0, st, oGroupStepOffset,
                       oUnitFirst, NG, P.unitSteps, oUnits);
    // partial-sum slots of the units of shared groups, and the shared groups
    std::uint32_t shared[2] = {};  // units with a slot, shared groups
    DevBuf<char> slotScratch;
    {
        const std::uint64_t n = std::max<std::uint64_t>(NU, NG) + 1;
        const std::size_t bytes = 4 * align_up(4 * n) + align_up(4 * scan_temp_elems(n)) + 256;
        if (hipMalloc(&slotScratch.p, bytes) != hipSuccess) {
            set_last_error("out of device memory for the hub tiles' partial slots");
            return fail(TCC_ERR_NO_MEMORY);
        }
        auto* groupShared = reinterpret_cast<std::uint32_t*>(slotScratch.p);
        auto* groupPos = reinterpret_cast<std::uint32_t*>(slotScratch.p + align_up(4 * n));
        auto* unitShared = reinterpret_cast<std::uint32_t*>(slotScratch.p + 2 * align_up(4 * n));
        auto* unitPos = reinterpret_cast<std::uint32_t*>(slotScratch.p + 3 * align_up(4 * n));
        auto* totals = reinterpret_cast<std::uint32_t*>(slotScratch.p + 4 * align_up(4 * n));
        auto* scanTemp = reinterpret_cast<std::uint32_t*>(slotScratch.p + 4 * align_up(4 * n) + 256);
        hipLaunchKernelGGL(shared_groups_kernel, dim3(grid_for(NG, kThreads)), dim3(kThreads), 0, st, oUnitFirst, NG,
                           groupShared);
        ok = exclusive_scan(groupShared, groupPos, NG, totals + 1, scanTemp, st) == hipSuccess;
        if (ok && NU > 0) {
            hipLaunchKernelGGL(shared_units_kernel, dim3(grid_for(NU, kThreads)), dim3(kThreads), 0, st, oUnits, NU,
                               groupShared, unitShared);
            ok = exclusive_scan(unitShared, unitPos, NU, totals, scanTemp, st) == hipSuccess;
            hipLaunchKernelGGL(partial_slots_kernel, dim3(grid_for(NU, kThreads)), dim3(kThreads), 0, st, NU,
                               unitShared, unitPos, oUnitPartial);
            hipLaunchKernelGGL(shared_group_list_kernel, dim3(grid_for(NG, kThreads)), dim3(kThreads), 0, st,
                               oUnitFirst, NG, groupShared, groupPos, unitPos, oSharedGroups);
        } else if (ok) {
            ok = fill<std::uint32_t>(totals, 1, 0u, st) == hipSuccess;
        }
        ok = ok && hipGetLastError() == hipSuccess &&
             hipMemcpyAsync(shared, totals, sizeof(shared), hipMemcpyDeviceToHost, st) == hipSuccess;
        if (!ok) {
            set_last_error("HIP error while numbering the hub tiles' partial sums");
            return fail(TCC_ERR_HIP);
        }
    }
    // launch order: units by the column block of their first step (stable);
    // binary tiles: the largest size bucket first
    DevBuf<char> orderScratch;
    if (NU > 0) {
        const std::uint64_t tempElems = radix_temp_elems(NU);
        const std::size_t bytes = align_up(16ull * NU) + align_up(4ull * NU) + align_up(4 * tempElems);
        if (hipMalloc(&orderScratch.p, bytes) != hipSuccess) {
            set_last_error("out of device memory for the hub tiles' unit order");
            return fail(TCC_ERR_NO_MEMORY);
        }
        auto* keys = reinterpret_cast<std::uint64_t*>(orderScratch.p);
        auto* vals = reinterpret_cast<std::uint32_t*>(orderScratch.p + align_up(16ull * NU));
        auto* sortTemp = reinterpret_cast<std::uint32_t*>(orderScratch.p + align_up(16ull * NU) + align_up(4ull * NU));
        unsigned bits = 0;
        while (bits < 32 && (static_cast<std::uint64_t>(CB) - 1) >> bits) ++bits;
        hipLaunchKernelGGL(unit_order_keys_kernel, dim3(grid_for(NU, kThreads)), dim3(kThreads), 0, st, oUnits, oStepCol,
                           NU, binary, bits, keys, oUnitOrder);
        if (binary) bits += 16;
        std::uint64_t* sortedKeys = nullptr;
        std::uint32_t* sortedOrder = nullptr;
        if (hipGetLastError() != hipSuccess ||
            radix_sort_pairs(keys, keys + NU, oUnitOrder, vals, NU, bits, sortTemp, &sortedKeys, &sortedOrder, st) !=
                hipSuccess ||
            (sortedOrder != oUnitOrder &&
             hipMemcpyAsync(oUnitOrder, sortedOrder, 4ull * NU, hipMemcpyDeviceToDevice, st) != hipSuccess)) {
            set_last_error("HIP error while ordering the hub tiles' units");
            return fail(TCC_ERR_HIP);
        }
    }
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        set_last_error("HIP error while building the hub tiles");
        return fail(TCC_ERR_HIP);
    }
    // the remainder: an ordinary or phased BCSR of the entries outside dense tiles
    tcc_bcsr rest{};
    void* restAlloc = nullptr;
    const float* rv = P.val ? restVal : nullptr;
    const int rc = tcc_coo_to_bcsr_phased(NR ? restRow : nullptr, NR ? restCol : nullptr, rv, NR, numRows, numCols,
                                          P.phases, &rest, &restAlloc, stream);
    if (rc) return fail(rc);
    rest.unitBlocks = kRestUnitBlocks;

    tcc_hub_tiles& T = out->tiles;
    T.num_rows = numRows;
    T.num_cols = numCols;
    T.nnz = E - NR;
    T.group_blocks = G;
    T.num_groups = NG;
    T.num_steps = NSS;
    T.num_tiles = ND;
    T.num_units = NU;
    T.unit_steps = P.unitSteps;
    T.hub_cols = hubCols;
    T.tile_format = P.format;
    T.rowOrder = oRowOrder;
    T.hubColOrder = oHubCols;
    T.groupStepOffset = oGroupStepOffset;
    T.stepCol = oStepCol;
    T.tileVals = oTileVals;
    T.units = oUnits;
    T.unitOrder = oUnitOrder;
    T.num_partial_units = NU > 0 ? shared[0] : 0;
    T.num_shared_groups = shared[1];
    T.unitPartial = oUnitPartial;
    T.sharedGroups = oSharedGroups;
    T.tileMasks = oTileMasks;
    T.rowScale = oRowScale;
    T.colScale = oColScale;
    out->rest = rest;
    out->tilesAllocation = o;
    out->restAllocation = restAlloc;
    out->restRowScale = oRestRowScale;
    return TCC_OK;
}

bool tiles_ok(const tcc_hub_tiles* T) {
    if (T->tile_format == TCC_TILES_BINARY)
        return valid_binary_group(T->group_blocks) && T->unit_steps >= 1 && T->tileMasks;
    return (T->tile_format == TCC_TILES_FP32 || T->tile_format == TCC_TILES_BF16X2) && valid_group(T->group_blocks) &&
           T->unit_steps >= 1 && T->unit_steps <= kMaxUnitSteps && T->tileVals;
}

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
                      std::uint32_t numRows, std::uint32_t numCols, std::uint32_t minTileNnz, std::uint32_t groupBlocks,
                      std::uint32_t unitSteps, std::uint32_t tileFormat, std::uint32_t phases, tcc_hybrid* out,
                      void* stream) {
    clear_last_error();
    TCC_REQUIRE(out && numRows >= 1 && numCols >= 1 && (nnz == 0 || (dRow && dCol)), TCC_ERR_INVALID_ARGUMENT,
                "invalid COO -> hybrid arguments");
    if (minTileNnz == 0) minTileNnz = kDefaultMinTileNnz;
    if (groupBlocks == 0) groupBlocks = kDefaultGroupBlocks;
    if (unitSteps == 0) unitSteps = kDefaultUnitSteps;
    TCC_REQUIRE(minTileNnz <= kTileVals, TCC_ERR_INVALID_ARGUMENT, "hybrid: minTileNnz above 256 leaves no tile");
    TCC_REQUIRE(valid_group(groupBlocks), TCC_ERR_INVALID_ARGUMENT, "hybrid: groupBlocks must be 1, 2, 4 or 8");
    TCC_REQUIRE(unitSteps <= kMaxUnitSteps, TCC_ERR_INVALID_ARGUMENT, "hybrid: unitSteps above 256");
    TCC_REQUIRE(tileFormat == TCC_TILES_FP32 || tileFormat == TCC_TILES_BF16X2, TCC_ERR_INVALID_ARGUMENT,
                "hybrid: tileFormat must be TCC_TILES_FP32 or TCC_TILES_BF16X2 (binary tiles: "
                "tcc_coo_to_hybrid_scaled)");
    HybridParams P{};
    P.row = dRow;
    P.col = dCol;
    P.val = dVal;
    P.nnz = nnz;
    P.numRows = numRows;
    P.numCols = numCols;
    P.minStepNnz = 0;
    P.minTileNnz = minTileNnz;
    P.G = groupBlocks;
    P.unitSteps = unitSteps;
    P.format = tileFormat;
    P.phases = phases;
    return build_hybrid(P, out, stream);
}

int tcc_coo_to_hybrid_scaled(const std::uint32_t* dRow, const std::uint32_t* dCol, std::uint32_t nnz,
                             std::uint32_t numRows, std::uint32_t numCols, const float* dRowScale,
                             const float* dColScale, std::uint32_t minStepNnz, std::uint32_t groupBlocks,
                             std::uint32_t unitSteps, std::uint32_t phases, tcc_hybrid* out, void* stream) {
    clear_last_error();
    TCC_REQUIRE(out && numRows >= 1 && numCols >= 1 && (nnz == 0 || (dRow && dCol)), TCC_ERR_INVALID_ARGUMENT,
                "invalid COO -> hybrid arguments");
    if (minStepNnz == 0) minStepNnz = kDefaultMinStepNnz;
    if (groupBlocks == 0) groupBlocks = kDefaultBinaryGroupBlocks;
    if (unitSteps == 0) unitSteps = kDefaultBinaryUnitSteps;
    TCC_REQUIRE(valid_binary_group(groupBlocks), TCC_ERR_INVALID_ARGUMENT,
                "hybrid: binary tiles take groupBlocks 8 or 16");
    HybridParams P{};
    P.row = dRow;
    P.col = dCol;
    P.nnz = nnz;
    P.numRows = numRows;
    P.numCols = numCols;
    P.minStepNnz = minStepNnz;
    P.minTileNnz = 1;  // every entry of a chosen step
    P.G = groupBlocks;
    P.unitSteps = unitSteps;
    P.format = TCC_TILES_BINARY;
    P.phases = phases;
    P.rowScale = dRowScale;
    P.colScale = dColScale;
    return build_hybrid(P, out, stream);
}

int tcc_hybrid_from_bcsr(const tcc_bcsr* A, int useValues, std::uint32_t minStepNnz, std::uint32_t phases,
                         tcc_hybrid* out, void* stream) {
    clear_last_error();
    TCC_REQUIRE(A && out && A->num_rows >= 1 && A->num_cols >= 1 && A->phases <= 1 &&
                    (A->num_TCBlocks == 0 || (A->rowWindowOffset && A->sparseA2B && A->tcLocalBit)) &&
                    (!useValues || (A->data && A->tcOffset)),
                TCC_ERR_INVALID_ARGUMENT, "invalid BCSR -> hybrid arguments (an ordinary BCSR; data for values)");
    const hipStream_t st = as_stream(stream);
    const std::uint32_t B = A->num_TCBlocks;
    // long windows take a phased remainder: 2 phases behind binary tiles
    // (config 3 step 4.76 ms against 4.99 with 4 and 4.79 with 1; the
    // remainder holds 9.8% of the entries), 4 behind value tiles (35%)
    if (phases == 0) phases = A->num_rowWindows && B >= 64ull * A->num_rowWindows ? (useValues ? 4 : 2) : 1;
    // block counts, their scan, then the entries
    DevBuf<char> scratch;
    const std::uint64_t Bn = std::max<std::uint32_t>(B, 1);
    const std::size_t headBytes = 2 * align_up(4 * (Bn + 1)) + align_up(4 * scan_temp_elems(Bn + 1)) + 256;
    TCC_HIP_CHECK(hipMalloc(&scratch.p, headBytes));
    auto* counts = reinterpret_cast<std::uint32_t*>(scratch.p);
    auto* offset = reinterpret_cast<std::uint32_t*>(scratch.p + align_up(4 * (Bn + 1)));
    auto* total = reinterpret_cast<std::uint32_t*>(scratch.p + 2 * align_up(4 * (Bn + 1)));
    auto* temp = reinterpret_cast<std::uint32_t*>(scratch.p + 2 * align_up(4 * (Bn + 1)) + 256);
    std::uint32_t E = 0;
    if (B > 0) {
        hipLaunchKernelGGL(bcsr_entry_counts_kernel, dim3(grid_for(B, kThreads)), dim3(kThreads), 0, st, *A, counts);
        TCC_LAUNCH_CHECK();
        TCC_HIP_CHECK(exclusive_scan(counts, offset, B, total, temp, st));
        TCC_HIP_CHECK(hipMemcpyAsync(&E, total, 4, hipMemcpyDeviceToHost, st));
        TCC_HIP_CHECK(hipStreamSynchronize(st));
    }
    DevBuf<char> coo;
    const std::uint64_t En = std::max<std::uint32_t>(E, 1);
    TCC_HIP_CHECK(hipMalloc(&coo.p, 3 * align_up(4 * En)));
    auto* row = reinterpret_cast<std::uint32_t*>(coo.p);
    auto* col = reinterpret_cast<std::uint32_t*>(coo.p + align_up(4 * En));
    auto* val = reinterpret_cast<float*>(coo.p + 2 * align_up(4 * En));
    if (E > 0) {
        hipLaunchKernelGGL(bcsr_expand_kernel, dim3(grid_for(B, kThreads)), dim3(kThreads), 0, st, *A, offset,
                           useValues != 0, row, col, val);
        TCC_LAUNCH_CHECK();
    }
    HybridParams P{};
    P.row = E ? row : nullptr;
    P.col = E ? col : nullptr;
    P.nnz = E;
    P.numRows = A->num_rows;
    P.numCols = A->num_cols;
    P.phases = phases;
    if (useValues) {
        P.val = val;
        P.minStepNnz = 0;
        P.minTileNnz = kDefaultMinTileNnz;
        P.G = kDefaultGroupBlocks;
        P.unitSteps = kDefaultUnitSteps;
        P.format = TCC_TILES_BF16X2;
    } else {
        P.minStepNnz = minStepNnz ? minStepNnz : kDefaultMinStepNnz;
        P.minTileNnz = 1;
        P.G = kDefaultBinaryGroupBlocks;
        P.unitSteps = kDefaultBinaryUnitSteps;
        P.format = TCC_TILES_BINARY;
    }
    return build_hybrid(P, out, stream);
}

// Binary tiles' half records: the per-workgroup maxima of hub_absmax_kernel,
// 2^e and 2^-e per slice, and a flag per (column block, slice).
constexpr std::uint32_t kAbsmaxBlocks = 2048;
constexpr std::uint32_t kMaxHalfSlices = kPackMaxSlices;

struct HalfSpace {
    std::size_t partial, up, down, flags, bytes;
};

inline HalfSpace half_space(std::uint32_t hubRows, std::uint32_t slices) {
    HalfSpace h;
    h.partial = 0;
    h.up = align_up(std::size_t(4) * kPackSliceMaxRows * slices);
    h.down = h.up + align_up(std::size_t(4) * slices);
    h.flags = h.down + align_up(std::size_t(4) * slices);
    h.bytes = h.flags + align_up(static_cast<std::size_t>(hubRows / kTile) * slices);
    return h;
}

size_t tcc_hub_tiles_workspace_bytes(const tcc_hub_tiles* T, std::uint32_t featureDim) {
    if (!T || featureDim == 0) return 0;
    const std::size_t ldh = hub_ldh(featureDim);
    std::size_t bytes = align_up(static_cast<size_t>(hub_rows(T)) * ldh * sizeof(float)) +
                        align_up(static_cast<size_t>(T->num_partial_units) * T->group_blocks * kTile * ldh * sizeof(float));
    const std::uint32_t slices = static_cast<std::uint32_t>(ldh / (32u * binary_nt(T->group_blocks)));
    if (T->tile_format == TCC_TILES_BINARY && slices <= kMaxHalfSlices)
        bytes += half_space(hub_rows(T), slices).bytes;
    return bytes;
}

size_t tcc_hybrid_workspace_bytes(const tcc_hybrid* H, std::uint32_t featureDim) {
    if (!H || featureDim == 0) return 0;
    return align_up(tcc_tf32_packed_bytes(H->rest.num_cols, featureDim) + 16) +
           tcc_hub_tiles_workspace_bytes(&H->tiles, featureDim);
}

// Where the slice maxima of binary tiles' half records sit in a tiles
// workspace, with the slice width and count (nullptr: bf16 records, no
// maxima).
static std::uint32_t* hub_slice_max(const tcc_hub_tiles* T, std::uint32_t featureDim, void* workspace,
                                    std::uint32_t& W, std::uint32_t& slices) {
    if (T->tile_format != TCC_TILES_BINARY) return nullptr;
    const std::uint32_t ldh = hub_ldh(featureDim);
    W = 32u * binary_nt(T->group_blocks);
    slices = ldh / W;
    if (slices > kMaxHalfSlices) return nullptr;
    const std::uint64_t n = static_cast<std::uint64_t>(hub_rows(T)) * ldh;
    char* halfBase = static_cast<char*>(workspace) + align_up(n * sizeof(float)) +
                     align_up(static_cast<size_t>(T->num_partial_units) * T->group_blocks * kTile * ldh * sizeof(float));
    return reinterpret_cast<std::uint32_t*>(halfBase + half_space(hub_rows(T), slices).partial);
}

// tcc_hub_tiles_spmm; maxReady: the slice maxima of half records are in the
// workspace already (the hybrid's remainder pack gathered them).
static int hub_tiles_spmm(const tcc_hub_tiles* T, const float* X, float* Y, std::uint32_t featureDim, void* workspace,
                          size_t workspaceBytes, void* stream, bool maxReady, bool storeY = false,
                          std::uint32_t outRows = 0) {
    TCC_REQUIRE(T && X && Y && featureDim >= 1 && T->rowOrder && T->groupStepOffset, TCC_ERR_INVALID_ARGUMENT,
                "invalid hub tiles SpMM arguments");
    if (T->num_units == 0) {
        // storeY: no unit writes any row
        if (storeY) TCC_HIP_CHECK(fill<float>(Y, static_cast<std::uint64_t>(outRows) * featureDim, 0.0f, as_stream(stream)));
        return TCC_OK;
    }
    TCC_REQUIRE(T->stepCol && T->units && T->hubColOrder && T->unitPartial &&
                    (T->num_shared_groups == 0 || T->sharedGroups),
                TCC_ERR_INVALID_ARGUMENT, "invalid hub tiles SpMM arguments");
    TCC_REQUIRE(tiles_ok(T), TCC_ERR_INVALID_ARGUMENT,
                "hub tiles: group_blocks must be 1, 2, 4 or 8 and unit_steps 1..256 (binary tiles: 8 or 16, any "
                "unit_steps), with the arrays of a known tile_format");
    const bool binary = T->tile_format == TCC_TILES_BINARY;
    const bool split = T->tile_format == TCC_TILES_BF16X2;
    const std::uint32_t ldh = hub_ldh(featureDim);
    TCC_REQUIRE(workspace && workspaceBytes >= tcc_hub_tiles_workspace_bytes(T, featureDim) &&
                    reinterpret_cast<std::uintptr_t>(workspace) % 16 == 0,
                TCC_ERR_INVALID_ARGUMENT, "hub tiles SpMM workspace too small or misaligned");
    const hipStream_t st = as_stream(stream);
    float* Xh = static_cast<float*>(workspace);
    const std::uint32_t hubRows = hub_rows(T);
    const std::uint64_t n = static_cast<std::uint64_t>(hubRows) * ldh;
    const std::uint32_t slices = ldh / (binary ? 32u * binary_nt(T->group_blocks) : kSlice);
    char* halfBase = static_cast<char*>(workspace) + align_up(n * sizeof(float)) +
                     align_up(static_cast<size_t>(T->num_partial_units) * T->group_blocks * kTile * ldh * sizeof(float));
    const HalfSpace hs = half_space(hubRows, slices);
    // Binary tiles take half records unless the slices' maxima would not fit
    // one workgroup's LDS (F above 2^19); then bf16 records throughout.
    const bool halfRecords = binary && slices <= kMaxHalfSlices;
    if (halfRecords) {
        // half records: each slice's scale from its largest magnitude, then
        // fp16 records where exact and bf16 halves elsewhere
        const std::uint32_t W = ldh / slices;
        std::uint32_t* partial = reinterpret_cast<std::uint32_t*>(halfBase + hs.partial);
        float* up = reinterpret_cast<float*>(halfBase + hs.up);
        float* down = reinterpret_cast<float*>(halfBase + hs.down);
        unsigned char* flags = reinterpret_cast<unsigned char*>(halfBase + hs.flags);
        if (!maxReady) {
            TCC_HIP_CHECK(fill<std::uint32_t>(partial, static_cast<std::uint64_t>(kPackSliceMaxRows) * slices, 0u, st));
            hipLaunchKernelGGL(hub_absmax_kernel, dim3(kAbsmaxBlocks), dim3(kThreads), slices * sizeof(std::uint32_t),
                               st, X, featureDim, T->hubColOrder, T->hub_cols, T->colScale, W, slices, partial);
            TCC_LAUNCH_CHECK();
        }
        hipLaunchKernelGGL(hub_scale_kernel, dim3(slices), dim3(kThreads), 0, st, partial, kPackSliceMaxRows, slices, up,
                           down);
        TCC_LAUNCH_CHECK();
        hipLaunchKernelGGL(hub_rows_half_kernel, dim3(grid_for(n / (2 * kTile), kThreads)), dim3(kThreads), 0, st, X,
                           featureDim, T->hubColOrder, T->hub_cols, hubRows, ldh, T->colScale, up, W,
                           reinterpret_cast<std::uint16_t*>(Xh), flags);
    } else if (split || binary) {
        hipLaunchKernelGGL(hub_rows_split_kernel, dim3(grid_for(n / kTile, kThreads)), dim3(kThreads), 0, st, X,
                           featureDim, T->hubColOrder, T->hub_cols, hubRows, ldh, binary ? T->colScale : nullptr,
                           reinterpret_cast<std::uint16_t*>(Xh));
    } else {
        const bool vecX = featureDim % 4 == 0 && (reinterpret_cast<std::uintptr_t>(X) & 15u) == 0;
        hipLaunchKernelGGL(hub_rows_kernel, dim3(grid_for(n / 4, kThreads)), dim3(kThreads), 0, st, X, featureDim,
                           T->hubColOrder, T->hub_cols, hubRows, ldh, vecX, Xh);
    }
    TCC_LAUNCH_CHECK();
    TileArgs a{};
    a.rowOrder = T->rowOrder;
    a.groupStepOffset = T->groupStepOffset;
    a.stepCol = T->stepCol;
    a.tileVals = T->tileVals;
    a.tileMasks = T->tileMasks;
    a.rowScale = binary ? T->rowScale : nullptr;
    a.units = T->units;
    a.unitPartial = T->unitPartial;
    a.sharedGroups = T->sharedGroups;
    a.unitOrder = T->unitOrder;
    a.Xh = Xh;
    a.ldh = ldh;
    a.Y = Y;
    a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + align_up(n * sizeof(float)));
    a.zeroStep = T->num_steps;
    a.F = featureDim;
    a.numUnits = T->num_units;
    a.slices = slices;
    a.storeY = storeY ? 1 : 0;
    a.zeroCol = binary ? hubRows / (2 * kTile) - 1 : 0;
    if (halfRecords) {
        a.halfFlags = reinterpret_cast<const unsigned char*>(halfBase + hs.flags);
        a.sliceDown = reinterpret_cast<const float*>(halfBase + hs.down);
    }
    const std::uint64_t waves = static_cast<std::uint64_t>(a.numUnits) * a.slices;
    TCC_REQUIRE(waves <= 0x7FFFFFFFull, TCC_ERR_UNSUPPORTED, "hub tiles SpMM launch too large");
    hipError_t e;
    if (binary) {
        e = launch_binary(a, T->group_blocks, st);
    } else {
        switch (T->group_blocks) {
            case 1: e = launch_tiles<1>(a, split, st); break;
            case 2: e = launch_tiles<2>(a, split, st); break;
            case 4: e = launch_tiles<4>(a, split, st); break;
            default: e = launch_tiles<8>(a, split, st); break;
        }
    }
    TCC_HIP_CHECK(e);
    if (storeY) {
        TCC_REQUIRE(outRows >= T->num_rows, TCC_ERR_INVALID_ARGUMENT, "hub tiles SpMM: fewer output rows than rows");
        const std::uint32_t numSlots = T->num_groups * T->group_blocks * kTile;
        const std::uint64_t waves = static_cast<std::uint64_t>(numSlots) + (outRows - T->num_rows);
        hipLaunchKernelGGL(hub_zero_rows_kernel, dim3(grid_for(waves * kWave, kThreads)), dim3(kThreads), 0, st, a,
                           T->group_blocks, numSlots, T->num_rows, outRows);
        TCC_LAUNCH_CHECK();
    }
    if (T->num_shared_groups == 0) return TCC_OK;
    const std::uint64_t reduceBlocks = static_cast<std::uint64_t>(T->num_shared_groups) * (ldh / kSlice) * T->group_blocks;
    TCC_REQUIRE(reduceBlocks <= 0x7FFFFFFFull, TCC_ERR_UNSUPPORTED, "hub tiles SpMM launch too large");
    hipLaunchKernelGGL(hub_reduce_kernel, dim3(static_cast<std::uint32_t>(reduceBlocks)), dim3(kThreads), 0, st, a,
                       T->group_blocks);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

int tcc_hub_tiles_spmm(const tcc_hub_tiles* T, const float* X, float* Y, std::uint32_t featureDim, void* workspace,
                       size_t workspaceBytes, void* stream) {
    clear_last_error();
    return hub_tiles_spmm(T, X, Y, featureDim, workspace, workspaceBytes, stream, false);
}

int tcc_hybrid_spmm(const tcc_hybrid* H, const float* X, float* Y, std::uint32_t featureDim, int accumulate,
                    void* workspace, size_t workspaceBytes, void* stream) {
    clear_last_error();
    TCC_REQUIRE(H && X && Y && featureDim >= 1 && workspace, TCC_ERR_INVALID_ARGUMENT, "invalid hybrid SpMM arguments");
    TCC_REQUIRE(workspaceBytes >= tcc_hybrid_workspace_bytes(H, featureDim) &&
                    reinterpret_cast<std::uintptr_t>(workspace) % 16 == 0,
                TCC_ERR_INVALID_ARGUMENT, "hybrid SpMM workspace too small or misaligned (tcc_hybrid_workspace_bytes)");
    // The remainder's product runs over packed TF32 rows when its rows are
    // gathered often (8 blocks per column on average, 16 gathers per row) or
    // its columns are scaled, else over X.  Binary tiles' scales apply to the
    // remainder too: column scales while packing, row scales to each row's
    // sum.  Binary tiles without accumulate run first and store their sums
    // (zeros in the rows no unit writes), and the remainder then adds into
    // Y: no zero fill of Y for the phased remainder's atomics, and no reads
    // of Y in the tiles' stores.  Otherwise the remainder writes (or adds
    // into) Y and the tiles add theirs.
    const bool binary = H->tiles.tile_format == TCC_TILES_BINARY;
    const float* colScale = binary ? H->tiles.colScale : nullptr;
    const float* rowScale = binary ? H->restRowScale : nullptr;
    const hipStream_t st = as_stream(stream);
    const std::uint64_t gathers = 8ull * H->rest.num_TCBlocks;
    const std::size_t packedBytes = align_up(tcc_tf32_packed_bytes(H->rest.num_cols, featureDim) + 16);
    const bool packs = colScale || gathers >= 16ull * H->rest.num_cols;
    int rc;
    // The tiles' half records take each slice's largest magnitude: the pack
    // of every column's scaled row gathers it on the way.
    void* tilesWs = static_cast<char*>(workspace) + packedBytes;
    const size_t tilesBytes = workspaceBytes - packedBytes;
    std::uint32_t W = 0, slices = 0;
    std::uint32_t* sliceMax = hub_slice_max(&H->tiles, featureDim, tilesWs, W, slices);
    bool maxReady = false;
    if (packs) {
        rc = tf32_pack_scaled(X, H->rest.num_cols, featureDim, colScale, workspace, st, sliceMax, W, slices);
        if (rc) return rc;
        maxReady = sliceMax != nullptr;
    }
    const bool tilesFirst = binary && !accumulate;
    if (tilesFirst) {
        const std::uint32_t outRows = H->rest.num_rowWindows / std::max(1u, H->rest.phases) * 8;
        rc = hub_tiles_spmm(&H->tiles, X, Y, featureDim, tilesWs, tilesBytes, stream, maxReady, true, outRows);
        if (rc) return rc;
    }
    const int restAccumulate = tilesFirst ? 1 : accumulate;
    rc = packs ? bcsr_spmm_packed_scaled(&H->rest, workspace, Y, featureDim, restAccumulate, rowScale, st)
               : bcsr_spmm_scaled(&H->rest, X, Y, featureDim, restAccumulate, rowScale, st);
    if (rc || tilesFirst) return rc;
    return hub_tiles_spmm(&H->tiles, X, Y, featureDim, tilesWs, tilesBytes, stream, maxReady);
}

}  // extern "C"
