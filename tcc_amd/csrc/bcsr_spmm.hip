// Block-sparse SpMM kernels behind spmm_cnic, for gfx950
// (reference: spmm_cnic/src/core/spmm_kernel.cu, spmm_dispatcher.cu,
// spmm_launcher.cu).
//
// Work split (merge-path over blocks): the blocks of a matrix are cut into
// units of K consecutive blocks, whatever the window boundaries, so every
// wave walks the same number of blocks however skewed the windows are (an
// R-MAT row window can hold thousands of blocks).  A wave finds the first
// window of its unit with a 64-way search over the window offsets, streams
// the block metadata, and finishes a window whenever its blocks end.  A
// window cut by a unit boundary is shared by several waves: its rows are
// zeroed first and every wave adds its partial sums with fp32 atomics; all
// other windows are stored directly.
//
// Gather (BCSR, mixed BCSR, BCSC read as A^T): one wave per (unit, chunk of
// 64*V features).  Each lane holds V consecutive features of the 8 output
// rows in registers.  Block metadata of 8 blocks is fetched with vector loads
// one group ahead (input-row pointers, bitmaps, value offsets) and read with
// v_readlane, so a block costs one round trip: its input rows (V-wide
// loads, rounded to TF32) and its values.  Nonzeros are walked with uniform
// branches over the bitmap: at the densities of the target graphs a block
// holds ~8 of its 64 entries, ~1 per column, so neither a dense 8x8 VALU
// contraction nor MFMA (which needs more than half the block set to beat
// FMA) pays off.
//
// Scatter (BCSC forward): one wave per (unit, chunk); the 8 source rows of
// the current window stay in registers and each block row is added into Y
// with fp32 atomics, as the reference does.
#include <algorithm>
#include <mutex>

#include "../../include/tcc_spmm_cnic.h"
#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "gather_ops.hpp"
#include "primitives.hpp"

namespace tcc {
namespace {

constexpr unsigned kThreads = 256;
constexpr unsigned kWaves = kThreads / kWave;
// Wave slots per compute unit (8 per SIMD).
constexpr std::uint32_t kMaxWaves = 32;

// Where a gather reads its input rows: fp32 X, the first layer's hot/cold
// feature source (fp32 or packed TF32 rows), dY for the A^T product, or a
// packed TF32 copy of X.
enum class Src { Plain, Mixed, MixedPacked, Transposed, Packed };

// Feature-source fields of the first GCN layer (tcc_feature_source).
struct MixedArgs {
    const std::int32_t* idMap;
    const std::int32_t* cacheSearchMap;
    const float* const* gpuCache;
    std::int32_t gpuNodeCapacity;
    const float* cpuFeatures;
    std::int64_t cpuLen;
    std::uint32_t gpuCacheCount;
    std::uint64_t rowBytes;  // 0: rows of F floats; else packed TF32 rows of this stride
    std::uint32_t* deviceError;  // receives TCC_DEVERR_FEATURE_INDEX on a refused lookup (or nullptr)
};

struct GatherArgs {
    const std::uint32_t* winOffset;  // [numWindows+1]
    const std::uint32_t* tcOffset;   // [blocks+1]
    const std::uint32_t* idx;        // [8*blocks] input row of each block column
    const std::uint64_t* bits;       // [blocks]
    const float* data;               // values or nullptr
    const float* X;                  // input rows (Plain / Transposed)
    const unsigned char* packed;     // packed TF32 rows (Packed)
    std::uint32_t packedStride;      // bytes per packed row
    float* Y;                        // [8*numWindows x F]
    std::uint32_t numWindows;
    std::uint32_t numBlocks;
    std::uint32_t numIn;  // idx values >= numIn are padding
    std::uint32_t F;
    std::uint32_t numChunks;
    std::uint32_t unitBlocks;
    std::uint32_t numUnits;
    int accumulate;
    int atomicOut;  // add every window into Y with atomics (Y zeroed by the caller)
    // Features [featureBase, featureEnd) of this launch (featureEnd 0 = F):
    // a packed gather launches its last, partial chunk on its own.
    std::uint32_t featureBase;
    std::uint32_t featureEnd;
    MixedArgs mixed;
    // Windows of the output (0: numWindows).  A phased matrix has `phases`
    // row windows per output window, window w adding into window w % outWindows.
    std::uint32_t outWindows;
    // Output row scales, or nullptr: row 8*ow + r of Y receives
    // rowScale[8*ow + r] * (its sum), so that A = diag(rowScale) * B for a
    // pattern (or valued) B; 8 entries per output window.
    const float* rowScale;
    // Rows of Y when it ends inside the last output window (0: 8 rows per
    // window), for adding into a Y of exactly the matrix's rows: rows at or
    // past it are neither read nor written (no window adds to them).
    std::uint32_t rowLimit;
};

// Feature row of column `in` for the first-layer (mixed) form
// (spmm_kernel.cu:129-153), or nullptr for a zero row: id_map < 0 (a column
// without a feature row), or a lookup outside its table, which is refused
// (read as zeros, and recorded in deviceError) instead of faulting.
__device__ __forceinline__ const float* table_row(const float* base, std::uint64_t rowBytes, std::uint32_t F,
                                                  std::int64_t r) {
    if (rowBytes == 0) return base + r * F;
    return reinterpret_cast<const float*>(reinterpret_cast<const unsigned char*>(base) + r * rowBytes);
}

__device__ __forceinline__ const float* refused(const MixedArgs& m) {
    if (m.deviceError) atomicOr(m.deviceError, TCC_DEVERR_FEATURE_INDEX);
    return nullptr;
}

__device__ __forceinline__ const float* mixed_row(const MixedArgs& m, std::uint32_t F, std::uint32_t in) {
    const std::int32_t g = m.cacheSearchMap[in];
    if (g >= 0) {
        const std::int32_t d = g / m.gpuNodeCapacity;
        if (m.gpuCacheCount != 0 && static_cast<std::uint32_t>(d) >= m.gpuCacheCount) return refused(m);
        return table_row(m.gpuCache[d], m.rowBytes, F, g % m.gpuNodeCapacity);
    }
    const std::int32_t id = m.idMap[in];
    if (id < 0) return nullptr;
    if (m.cpuFeatures == nullptr) return refused(m);
    if (m.cpuLen > 0 && (static_cast<std::int64_t>(id) + 1) * F > m.cpuLen) return refused(m);
    return table_row(m.cpuFeatures, m.rowBytes, F, id);
}

template <int V>
struct Vec {
    float v[V];
};

// Packed feature rows are read with 32-bit byte offsets from a row base
// (buffer loads): F below 2^30 keeps a packed row (2.5 bytes a feature), and
// an fp32 one, below 4 GiB.
constexpr bool feature_dim_ok(std::uint32_t F) { return F >= 1 && F < (1u << 30); }

template <int V>
__device__ __forceinline__ Vec<V> load_vec(const float* p) {
    Vec<V> r;
    if constexpr (V == 4) {
        const vf4 t = load_global<vf4>(p);
        r.v[0] = t.x; r.v[1] = t.y; r.v[2] = t.z; r.v[3] = t.w;
    } else if constexpr (V == 2) {
        const vf2 t = load_global<vf2>(p);
        r.v[0] = t.x; r.v[1] = t.y;
    } else {
        r.v[0] = load_global<float>(p);
    }
    return r;
}

template <int V>
__device__ __forceinline__ void store_vec(float* p, const float* v) {
    if constexpr (V == 4) {
        *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    } else if constexpr (V == 2) {
        *reinterpret_cast<float2*>(p) = make_float2(v[0], v[1]);
    } else {
        *p = v[0];
    }
}

// 8x8 bit-matrix transpose: bit (r*8+c) -> bit (c*8+r) (delta swaps).
__device__ __forceinline__ std::uint64_t transpose8x8(std::uint64_t x) {
    std::uint64_t t;
    t = (x ^ (x >> 7)) & 0x00AA00AA00AA00AAull;
    x = x ^ t ^ (t << 7);
    t = (x ^ (x >> 14)) & 0x0000CCCC0000CCCCull;
    x = x ^ t ^ (t << 14);
    t = (x ^ (x >> 28)) & 0x00000000F0F0F0F0ull;
    x = x ^ t ^ (t << 28);
    return x;
}

__device__ __forceinline__ std::uint32_t lane_u32(std::uint32_t v, int l) {
    return static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}

__device__ __forceinline__ std::uint32_t uniform(std::uint32_t v) {
    return static_cast<std::uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v)));
}

// First index i in [0, n) with off[i] >= key (n if there is none), for a
// non-decreasing off[], computed by one wave: each round probes 64 evenly
// spaced entries with one vector load and narrows the range to the gap the
// ballot points at (3 rounds for 2^18 entries).
__device__ std::uint32_t wave_lower_bound(const std::uint32_t* off, std::uint32_t n, std::uint32_t key) {
    const unsigned lane = __lane_id();
    std::uint32_t lo = 0, hi = n;  // answer in [lo, hi]
    while (hi - lo > 64) {
        const std::uint32_t step = (hi - lo + 63) / 64;
        const std::uint32_t p = lo + (lane + 1) * step - 1;
        const bool ge = p >= hi || off[p] >= key;
        const std::uint64_t m = __ballot(ge);
        if (m == 0) return hi;
        const std::uint32_t L = static_cast<std::uint32_t>(__builtin_ctzll(m));
        const std::uint32_t pL = lo + (L + 1) * step - 1;
        lo = lo + L * step;
        hi = min(pL, hi);
    }
    const std::uint32_t p = lo + lane;
    const bool ge = p >= hi || off[p] >= key;
    const std::uint64_t m = __ballot(ge);
    return m == 0 ? hi : lo + static_cast<std::uint32_t>(__builtin_ctzll(m));
}

// The blocks [b0, b1) of unit u and the first window it finishes: the
// window holding block b0, or (when windows start exactly at b0) the first
// of them, empty ones included.
struct UnitRange {
    std::uint32_t b0, b1, w;
    bool last;
};

__device__ __forceinline__ UnitRange unit_range(const std::uint32_t* winOffset, std::uint32_t numWindows,
                                                std::uint32_t numBlocks, std::uint32_t K, std::uint32_t numUnits,
                                                std::uint32_t u) {
    UnitRange r;
    r.b0 = u * K;
    r.b1 = min(r.b0 + K, numBlocks);
    r.last = u + 1 == numUnits;
    const std::uint32_t lb = uniform(wave_lower_bound(winOffset, numWindows + 1, r.b0));
    r.w = (lb <= numWindows && winOffset[lb] == r.b0) ? lb : lb - 1;
    return r;
}

// Row base pointer of input `in` (nullptr for a zero row).
template <Src MODE>
__device__ __forceinline__ const float* input_row(const GatherArgs& a, std::uint32_t in) {
    if constexpr (MODE == Src::Mixed || MODE == Src::MixedPacked) {
        return mixed_row(a.mixed, a.F, in);
    } else if constexpr (MODE == Src::Packed) {
        return reinterpret_cast<const float*>(a.packed + static_cast<std::uint64_t>(in) * a.packedStride);
    } else {
        return a.X + static_cast<std::uint64_t>(in) * a.F;
    }
}

// Packed TF32 rows (tcc_tf32_pack): a TF32 value has 19 significant bits,
// stored as its high 16 bits (sign, exponent, 7 mantissa bits) and its 3 low
// mantissa bits.  A row is cut into chunks of 256 features (the 64 lanes x 4
// features one wave gathers); a chunk of n features holds the high halves
// (2 bytes each) and then the low bits of element pairs (element 2k in bits
// 0-2 and 2k+1 in bits 3-5 of byte k): a full chunk is 640 bytes, five
// 128-byte lines, so a wave's chunk load touches exactly the lines it uses
// once rows are 128-byte aligned.  The last chunk is padded to 16 bytes and
// rows longer than one chunk to 128 bytes (single-chunk rows to 16).
// Exact: unpacking gives the TF32 rounding of X bit for bit.
constexpr std::uint32_t kPackChunk = 256;
constexpr std::uint64_t kPackChunkBytes = 640;

__host__ __device__ constexpr std::uint64_t packed_tail_bytes(std::uint32_t n) {
    return ((2ull * n + (n + 1) / 2) + 15) & ~15ull;
}

__host__ __device__ constexpr std::uint64_t packed_stride(std::uint32_t F) {
    const std::uint64_t full = F / kPackChunk, tail = F % kPackChunk;
    const std::uint64_t bytes = full * kPackChunkBytes + (tail ? packed_tail_bytes(static_cast<std::uint32_t>(tail)) : 0);
    return F > kPackChunk ? ((bytes + 127) & ~127ull) : bytes;
}

// Byte offsets of element f's high half and of the low-bit byte of its pair.
struct PackedAt {
    std::uint64_t hi, lo;
};

__host__ __device__ inline PackedAt packed_at(std::uint32_t F, std::uint32_t f) {
    const std::uint32_t c = f / kPackChunk, j = f % kPackChunk;
    const std::uint32_t n = (F - c * kPackChunk) < kPackChunk ? (F - c * kPackChunk) : kPackChunk;
    const std::uint64_t base = c * kPackChunkBytes;
    return PackedAt{base + 2ull * j, base + 2ull * n + j / 2};
}

__device__ __forceinline__ float tf32_from(std::uint32_t hi16, std::uint32_t lo3) {
    return __uint_as_float((hi16 << 16) | (lo3 << 13));
}

// The V features at element offset `f` of a packed row (f % V == 0; the V
// elements lie in one chunk): the high halves and the low bits, loaded
// before any use.  Elements past F read padding and are never stored.
template <int V>
struct PackedVec {
    std::uint32_t hi[(V + 1) / 2];
    std::uint32_t lo;
};

// Word 3 of a buffer resource on gfx9-family GPUs (raw, untyped access).
constexpr int kBufferWord3 = 0x00020000;

// Packed row `rp` as a buffer resource, `records` = ~0 for a row and 0 for
// none (rp and records wave-uniform, read with readlane, so the resource
// sits in scalar registers): loads then take the row base from scalar
// registers and a 32-bit lane offset, with no 64-bit address add per lane
// and load, and a missing row's loads return zeros without touching memory
// (a buffer load past num_records reads nothing), with no branch around
// them.  A packed row is below 4 GiB (feature_dim_ok).
template <int V>
__device__ __forceinline__ PackedVec<V> load_packed(std::uint64_t rp, std::uint32_t records, std::uint32_t F,
                                                    std::uint32_t f) {
    PackedVec<V> p;
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(rp), 0, static_cast<int>(records), kBufferWord3);
    const PackedAt at = packed_at(F, f);
    const int hi = static_cast<int>(at.hi), lo = static_cast<int>(at.lo);
    if constexpr (V == 4) {
        const vu2 h = __builtin_amdgcn_raw_buffer_load_b64(r, hi, 0, 0);
        p.hi[0] = h.x;
        p.hi[1] = h.y;
        p.lo = __builtin_amdgcn_raw_buffer_load_b16(r, lo, 0, 0);
    } else if constexpr (V == 2) {
        p.hi[0] = __builtin_amdgcn_raw_buffer_load_b32(r, hi, 0, 0);
        p.lo = __builtin_amdgcn_raw_buffer_load_b8(r, lo, 0, 0);
    } else {
        p.hi[0] = __builtin_amdgcn_raw_buffer_load_b16(r, hi, 0, 0);
        p.lo = static_cast<std::uint32_t>(__builtin_amdgcn_raw_buffer_load_b8(r, lo, 0, 0)) >> (3 * (f & 1u));
    }
    return p;
}

template <int V>
__device__ __forceinline__ void unpack(const PackedVec<V>& p, float* x) {
    if constexpr (V == 1) {
        x[0] = tf32_from(p.hi[0] & 0xFFFFu, p.lo & 7u);
    } else {
#pragma unroll
        for (int j = 0; j < V; ++j) {
            const std::uint32_t h = p.hi[j / 2];
            const std::uint32_t hi16 = (j & 1) ? (h >> 16) : (h & 0xFFFFu);
            x[j] = tf32_from(hi16, (p.lo >> (8 * (j / 2) + 3 * (j & 1))) & 7u);
        }
    }
}

// Metadata of up to 8 consecutive blocks g..g+7, gathered with vector loads
// one group ahead of its use: lane 8*k + c holds the input-row pointer of
// column c of block g+k (null for padding or a missing row); lanes 0..7 hold
// the bitmap and the value offset of block g+lane.
struct GroupMeta {
    std::uint32_t rowLo, rowHi;
    std::uint32_t rowRecords;  // ~0 where the lane's row exists, else 0 (the packed rows' buffer bound)
    std::uint32_t bitsLo, bitsHi;
    std::uint32_t off;
};

template <Src MODE, bool VALUES>
__device__ __forceinline__ GroupMeta load_group(const GatherArgs& a, std::uint32_t g, std::uint32_t end) {
    const unsigned lane = __lane_id();
    GroupMeta m;
    const float* row = nullptr;
    const std::uint32_t blk = g + lane / 8;
    if (blk < end) {
        const std::uint32_t in = a.idx[static_cast<std::uint64_t>(blk) * 8 + (lane & 7u)];
        if (in < a.numIn) row = input_row<MODE>(a, in);
    }
    const std::uint64_t rp = reinterpret_cast<std::uint64_t>(row);
    m.rowLo = static_cast<std::uint32_t>(rp);
    m.rowHi = static_cast<std::uint32_t>(rp >> 32);
    m.rowRecords = row ? ~0u : 0u;
    const std::uint32_t bb = g + (lane & 7u);
    std::uint64_t bits = 0;
    std::uint32_t off = 0;
    if (lane < 8 && bb < end) {
        bits = a.bits[bb];
        if constexpr (VALUES) off = a.tcOffset[bb];
    }
    m.bitsLo = static_cast<std::uint32_t>(bits);
    m.bitsHi = static_cast<std::uint32_t>(bits >> 32);
    m.off = off;
    return m;
}

// Block k of the group: its stored bitmap `raw`, the row-major view `bm`
// (byte R = the input columns C that output row R uses), the input rows x[C]
// (zeros for padding) and its values (lane i = the value of its i-th stored
// nonzero), TF32-rounded except for the A^T gather.  issue_block starts the
// loads, finish_block uses them; load_block does both.
template <int V, Src MODE>
struct BlockLoad {
    std::uint64_t raw;
    float vals;
    PackedVec<V> pk[8];  // packed sources
    float x[8][V];       // fp32 sources
};

template <int V, Src MODE, bool VALUES>
__device__ __forceinline__ void issue_block(const GatherArgs& a, const GroupMeta& m, int k, std::uint32_t laneOff,
                                            BlockLoad<V, MODE>& b) {
    b.raw = (static_cast<std::uint64_t>(lane_u32(m.bitsHi, k)) << 32) | lane_u32(m.bitsLo, k);
    // All loads are issued before any result is used (rounding inside the
    // branches would wait for each load in turn).
    if constexpr (MODE == Src::Packed || MODE == Src::MixedPacked) {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const std::uint64_t rp = (static_cast<std::uint64_t>(lane_u32(m.rowHi, k * 8 + c)) << 32) |
                                     lane_u32(m.rowLo, k * 8 + c);
            b.pk[c] = load_packed<V>(rp, lane_u32(m.rowRecords, k * 8 + c), a.F, laneOff);
        }
    } else {
        // fp32 rows keep 64-bit addresses and a branch per missing row: the
        // buffer form of the packed rows measured slower here (config 5's
        // first layer, hot and host rows: 12.0 against 11.7 ms per pass).
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const std::uint64_t rp = (static_cast<std::uint64_t>(lane_u32(m.rowHi, k * 8 + c)) << 32) |
                                     lane_u32(m.rowLo, k * 8 + c);
#pragma unroll
            for (int v = 0; v < V; ++v) b.x[c][v] = 0.0f;
            if (rp != 0) {
                const Vec<V> t = load_vec<V>(reinterpret_cast<const float*>(rp) + laneOff);
#pragma unroll
                for (int v = 0; v < V; ++v) b.x[c][v] = t.v[v];
            }
        }
    }
    b.vals = 0.0f;
    if constexpr (VALUES) {
        const std::uint32_t off = lane_u32(m.off, k);
        if (__lane_id() < static_cast<unsigned>(__popcll(b.raw))) b.vals = a.data[off + __lane_id()];
    }
}

template <int V, Src MODE, bool VALUES>
__device__ __forceinline__ void finish_block(const BlockLoad<V, MODE>& b, std::uint64_t& bm, float (&x)[8][V],
                                             float& vals) {
    // Stored bit (r*8+c): BCSR = (output row r, column c); BCSC = (source row r,
    // source column c), i.e. (input r, output c) for the A^T gather.
    bm = (MODE == Src::Transposed) ? transpose8x8(b.raw) : b.raw;
    if constexpr (MODE == Src::Packed || MODE == Src::MixedPacked) {
#pragma unroll
        for (int c = 0; c < 8; ++c) unpack<V>(b.pk[c], x[c]);
    } else {
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int v = 0; v < V; ++v) x[c][v] = b.x[c][v];
    }
    vals = b.vals;
    // The A^T product replaces torch.sparse.mm in the reference's backward
    // (train/tcgnn_conv_release.py:152), which multiplies in plain fp32; the
    // forward products reproduce its mma.m16n8k8 tf32 numerics (packed rows
    // hold TF32 values already).
    if constexpr (MODE == Src::Plain || MODE == Src::Mixed) {
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int v = 0; v < V; ++v) x[c][v] = tf32_rna(x[c][v]);
    }
    if constexpr (VALUES && MODE != Src::Transposed) vals = tf32_rna(vals);
}

template <int V, Src MODE, bool VALUES>
__device__ __forceinline__ void load_block(const GatherArgs& a, const GroupMeta& m, int k, std::uint32_t laneOff,
                                           std::uint64_t& raw, std::uint64_t& bm, float (&x)[8][V], float& vals) {
    BlockLoad<V, MODE> b;
    issue_block<V, MODE, VALUES>(a, m, k, laneOff, b);
    finish_block<V, MODE, VALUES>(b, bm, x, vals);
    raw = b.raw;
}

// acc[R] += w(R,C) * x[C] over the block's nonzeros (uniform branches over
// the bitmap); w = 1 without values, else the value whose rank is the number
// of stored nonzeros below its bit, read from `vals` with v_readlane.
template <int V, Src MODE, bool VALUES>
__device__ __forceinline__ void accumulate_block(std::uint64_t raw, std::uint64_t bm, float vals,
                                                 const float (&x)[8][V], float (&acc)[8][V]) {
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        const std::uint32_t rb = static_cast<std::uint32_t>(bm >> (8 * r)) & 0xFFu;
        if (rb == 0) continue;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if (!(rb & (1u << c))) continue;
            if constexpr (!VALUES) {
#pragma unroll
                for (int v = 0; v < V; ++v) acc[r][v] += x[c][v];
            } else {
                const unsigned stored = (MODE == Src::Transposed) ? (c * 8 + r) : (r * 8 + c);
                const int rank = static_cast<int>(__popcll(raw & ((1ull << stored) - 1ull)));
                const float w = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vals), rank));
#pragma unroll
                for (int v = 0; v < V; ++v) acc[r][v] = fmaf(w, x[c][v], acc[r][v]);
            }
        }
    }
}

// One wave per (unit, feature chunk of 64*V); waves are ordered chunk-major
// so that the input rows one chunk touches stay in the last-level cache.
template <int V, Src MODE, bool VALUES>
__device__ __forceinline__ void gather_body(const GatherArgs& a, std::uint32_t gw) {
    const unsigned lane = __lane_id();
    const std::uint32_t chunk = gw / a.numUnits;
    const std::uint32_t unit = gw - chunk * a.numUnits;
    if (chunk >= a.numChunks) return;
    const UnitRange u = unit_range(a.winOffset, a.numWindows, a.numBlocks, a.unitBlocks, a.numUnits, unit);
    if (u.w >= a.numWindows) return;  // offsets inconsistent with the block count
    const std::uint32_t f0 = a.featureBase + chunk * (kWave * V) + lane * V;
    const bool active = f0 < (a.featureEnd ? a.featureEnd : a.F);
    // Inactive lanes read lane 0's features (active, so in bounds, and on
    // the lines the wave loads anyway) and never store.  Reading the row
    // start instead fetched two more lines per row in a tail launch
    // (features 512-601 of config 3: 13.5 GB fetched for about 10 GB).
    const std::uint32_t laneOff = active ? f0 : f0 - lane * V;

    __shared__ float flushStage[V == 4 ? kWaves * kWave * V : 1];
    float acc[8][V];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int v = 0; v < V; ++v) acc[r][v] = 0.0f;
    std::uint64_t touched = 0;  // union of the current window's row-major bitmaps

    std::uint32_t w = u.w;
    std::uint32_t ws = a.winOffset[w], we = a.winOffset[w + 1];
    // Finish window w: a window cut by a unit boundary is shared (rows
    // pre-zeroed unless accumulating; atomics for the rows this unit
    // touched), any other is stored whole.
    // V-wide stores when F % V == 0 (then rows keep V-float alignment), else
    // (the packed gather's 4-wide chunks over any F) one float at a time.
    // Only the packed sources pick V without F % V == 0.
    constexpr bool kWhole = MODE != Src::Packed && MODE != Src::MixedPacked;
    const bool vecStore = kWhole || a.F % V == 0;
    auto flush = [&]() {
        const std::uint32_t ow = a.outWindows ? w % a.outWindows : w;
        const bool shared = a.atomicOut || ws < u.b0 || we > u.b1;  // wave-uniform
        if (a.rowScale) {
            // the window's 8 row scales (wave-uniform loads), applied to the
            // partial sum before it is stored or added
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const float s = a.rowScale[static_cast<std::uint64_t>(ow) * 8 + r];
#pragma unroll
                for (int v = 0; v < V; ++v) acc[r][v] *= s;
            }
        }
        if (V == 4 && shared) {
            // A row's 256 sums pass through LDS so that each atomic
            // instruction adds 64 consecutive floats (lane l: feature
            // 64j + l of the chunk) rather than every 4th float of 1 KB: a
            // quarter of the L2 requests.  On config 3 with every window
            // added atomically, 20.7 -> 19.9 ms.  (At V = 2 the staging
            // costs the 64-VGPR kernels a wave per SIMD.)  Every lane takes
            // part, active or not: lane l adds the features below the
            // launch's end, whose owners (lane (64j + l) / 4) are active.
            float* st = flushStage + uniform(threadIdx.x / kWave) * (kWave * V);
            const std::uint32_t cb = f0 - lane * V;
            const std::uint32_t fe = a.featureEnd ? a.featureEnd : a.F;
            float* rb = a.Y + static_cast<std::uint64_t>(ow) * 8 * a.F + cb;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                if (((touched >> (8 * r)) & 0xFFu) == 0) continue;
                store_vec<V>(st + lane * V, acc[r]);
                __builtin_amdgcn_wave_barrier();
                float t[V];
#pragma unroll
                for (int j = 0; j < V; ++j) t[j] = st[kWave * j + lane];
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int j = 0; j < V; ++j)
                    if (cb + kWave * j + lane < fe)
                        atomic_add_f32(rb + static_cast<std::uint64_t>(r) * a.F + kWave * j + lane, t[j]);
            }
        } else if (active) {
            float* out = a.Y + static_cast<std::uint64_t>(ow) * 8 * a.F + f0;
            // rows of the window inside Y (wave-uniform; 8 but in a last
            // window cut by rowLimit, whose rows past it read row 0)
            const std::uint32_t live = a.rowLimit ? min(8u, a.rowLimit - ow * 8) : 8u;
            if (!shared && vecStore && a.accumulate) {
                // Y += : all 8 rows loaded before any is added
                Vec<V> prev[8];
#pragma unroll
                for (int r = 0; r < 8; ++r)
                    prev[r] = load_vec<V>(out + static_cast<std::uint64_t>(r < static_cast<int>(live) ? r : 0) * a.F);
#pragma unroll
                for (int r = 0; r < 8; ++r)
#pragma unroll
                    for (int v = 0; v < V; ++v) acc[r][v] += prev[r].v[v];
            }
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                float* o = out + static_cast<std::uint64_t>(r) * a.F;
                if (shared) {
                    if (((touched >> (8 * r)) & 0xFFu) == 0) continue;
#pragma unroll
                    for (int v = 0; v < V; ++v)
                        if (kWhole || f0 + v < a.F) atomic_add_f32(o + v, acc[r][v]);
                } else if (r >= static_cast<int>(live)) {
                    continue;
                } else if (vecStore) {
                    store_vec<V>(o, acc[r]);
                } else {
#pragma unroll
                    for (int v = 0; v < V; ++v)
                        if (f0 + v < a.F) o[v] = a.accumulate ? o[v] + acc[r][v] : acc[r][v];
                }
            }
        }
#pragma unroll
        for (int r = 0; r < 8; ++r)
#pragma unroll
            for (int v = 0; v < V; ++v) acc[r][v] = 0.0f;
        touched = 0;
    };

    GroupMeta cur = load_group<MODE, VALUES>(a, u.b0, u.b1);
    for (std::uint32_t g = u.b0; g < u.b1; g += 8) {
        GroupMeta nxt = cur;
        if (g + 8 < u.b1) nxt = load_group<MODE, VALUES>(a, g + 8, u.b1);
        const int nb = static_cast<int>(min(8u, u.b1 - g));
        for (int k = 0; k < nb; ++k) {
            while (g + k >= we && w + 1 < a.numWindows) {  // the window ends before this block
                flush();
                ++w;
                ws = we;
                we = a.winOffset[w + 1];
            }
            std::uint64_t raw, bm;
            float x[8][V], vv;
            load_block<V, MODE, VALUES>(a, cur, k, laneOff, raw, bm, x, vv);
            accumulate_block<V, MODE, VALUES>(raw, bm, vv, x, acc);
            touched |= bm;
        }
        cur = nxt;
    }
    flush();
    if (u.last) {
        // trailing empty windows (offset == number of blocks)
        while (++w < a.numWindows) {
            ws = we = u.b1;
            flush();
        }
    }
}

template <int V, Src MODE, bool VALUES>
__global__ void __launch_bounds__(kThreads) gather_kernel(GatherArgs a) {
    gather_body<V, MODE, VALUES>(a, blockIdx.x * kWaves + uniform(threadIdx.x / kWave));
}

// Zero the rows of every window a unit boundary cuts (so that the units
// sharing it can add into them).  Window [s, e) holds a boundary (a multiple
// of K) strictly inside iff (s / K + 1) * K < e, so one lane per window
// decides from its two offsets, with no search; each wave then zeroes its
// cut windows together, 16 bytes a lane (a window's 8 rows are one block of
// 8F floats).  One lane per boundary searching for its window took 6.2 us
// on config 2 (4,834 boundaries), a three-load search chain per wave.
__global__ void __launch_bounds__(kThreads) zero_shared_windows_kernel(const std::uint32_t* __restrict__ winOffset,
                                                                      std::uint32_t numWindows, std::uint32_t K,
                                                                      float* __restrict__ Y, std::uint32_t F) {
    const std::uint32_t w = blockIdx.x * kThreads + threadIdx.x;
    bool cut = false;
    if (w < numWindows) {
        const std::uint32_t s = winOffset[w], e = winOffset[w + 1];
        cut = static_cast<std::uint64_t>(s / K + 1) * K < e;
    }
    std::uint64_t m = __ballot(cut);
    const std::uint32_t w0 = w - __lane_id();
    const bool vec = (reinterpret_cast<std::uintptr_t>(Y) & 15u) == 0;
    while (m) {
        const unsigned k = static_cast<unsigned>(__builtin_ctzll(m));
        m &= m - 1;
        float* p = Y + static_cast<std::uint64_t>(w0 + k) * 8 * F;
        if (vec) {
            float4* q = reinterpret_cast<float4*>(p);
            for (std::uint32_t i = __lane_id(); i < 2u * F; i += kWave) q[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        } else {
            for (std::uint32_t i = __lane_id(); i < 8u * F; i += kWave) p[i] = 0.0f;
        }
    }
}

// ------------------------------------------------------------ narrow gather
// Gather for F <= 16 (the GCN's class-width products A(XW) and A^T dY).  One
// wave per 64*V features would leave all but F lanes idle and pay a memory
// round trip per block; here a wave takes 8 blocks per step instead.  Lane
// 8k+j loads column j of block k (its input row, F features) and computes
// output row j of block k from the 8 column values of block k, exchanged
// within the 8-lane group with ds_swizzle.  Window sums stay in registers
// per (block slot, row) and are reduced across the 8 slots when the window
// ends.  Metadata is fetched two groups ahead and input rows one group
// ahead.  Y is zero-filled first (or accumulated into), so empty windows
// need no work and shared windows take atomics without a zeroing pass.

// Column j of block g+k (lane 8k+j) and block g+k's bitmap / value offset.
struct NarrowMeta {
    std::uint32_t in;  // >= numIn: padding or past the unit
    std::uint32_t bitsLo, bitsHi;
    std::uint32_t off;
};

template <bool VALUES>
__device__ __forceinline__ NarrowMeta narrow_meta(const GatherArgs& a, std::uint32_t g, std::uint32_t end) {
    const unsigned lane = __lane_id();
    const std::uint32_t b = g + (lane >> 3);
    NarrowMeta m{0xFFFFFFFFu, 0u, 0u, 0u};
    if (b < end) {
        m.in = a.idx[static_cast<std::uint64_t>(b) * 8 + (lane & 7u)];
        const std::uint64_t raw = a.bits[b];
        m.bitsLo = static_cast<std::uint32_t>(raw);
        m.bitsHi = static_cast<std::uint32_t>(raw >> 32);
        if constexpr (VALUES) m.off = a.tcOffset[b];
    }
    return m;
}

// Input row `in` (FT >= F features, zeros past F and for a missing row),
// with V-wide loads when F == FT and X is aligned for them (`vec`).
template <int FT, Src MODE>
__device__ __forceinline__ void narrow_row(const GatherArgs& a, std::uint32_t in, bool vec, float (&x)[FT]) {
#pragma unroll
    for (int f = 0; f < FT; ++f) x[f] = 0.0f;
    if (in >= a.numIn) return;
    const float* row = a.X + static_cast<std::uint64_t>(in) * a.F;
    if (vec) {
        constexpr int V = FT < 4 ? FT : 4;
#pragma unroll
        for (int f = 0; f < FT; f += V) {
            const Vec<V> t = load_vec<V>(row + f);
#pragma unroll
            for (int v = 0; v < V; ++v) x[f + v] = t.v[v];
        }
    } else {
#pragma unroll
        for (int f = 0; f < FT; ++f)
            if (static_cast<std::uint32_t>(f) < a.F) x[f] = row[f];
    }
}

// p += w(j, C) * x(column C of this lane's block), for C = 0..7: the column
// values come from lane (lane & ~7) | C (ds_swizzle bit mode inside each
// 32-lane half: and-mask 0x18 keeps the block slot, or-mask C picks the lane).
template <int C, int FT, bool VALUES>
__device__ __forceinline__ void narrow_columns(const float (&x)[FT], std::uint32_t rb, const float (&wv)[8],
                                               float (&p)[FT]) {
    float xc[FT];
#pragma unroll
    for (int f = 0; f < FT; ++f) xc[f] = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x[f]), 0x18 | (C << 5)));
    if ((rb >> C) & 1u) {
#pragma unroll
        for (int f = 0; f < FT; ++f) p[f] = VALUES ? fmaf(wv[C], xc[f], p[f]) : p[f] + xc[f];
    }
    if constexpr (C < 7) narrow_columns<C + 1, FT, VALUES>(x, rb, wv, p);
}

template <int FT, Src MODE, bool VALUES>
__global__ void __launch_bounds__(kThreads) narrow_gather_kernel(GatherArgs a) {
    const unsigned lane = __lane_id();
    const unsigned slot = lane >> 3, j = lane & 7u;
    const std::uint32_t unit = blockIdx.x * kWaves + uniform(threadIdx.x / kWave);
    if (unit >= a.numUnits) return;
    const UnitRange u = unit_range(a.winOffset, a.numWindows, a.numBlocks, a.unitBlocks, a.numUnits, unit);
    if (u.b0 >= u.b1 || u.w >= a.numWindows) return;
    constexpr int VA = FT < 4 ? FT : 4;
    const bool vec = a.F == FT && (reinterpret_cast<std::uintptr_t>(a.X) % (4u * VA)) == 0;

    // Window ends one vector load at a time: lane i holds winOffset[cbase+1+i]
    // (all ones past the last window), cstart = winOffset[cbase].
    std::uint32_t cbase = u.w, cstart = a.winOffset[u.w];
    auto load_ends = [&]() {
        const std::uint32_t i = cbase + 1 + lane;
        return i <= a.numWindows ? a.winOffset[i] : 0xFFFFFFFFu;
    };
    std::uint32_t ends = load_ends();
    std::uint32_t w = 0, ws = 0, we = 0;
    // The window holding block b (empty windows skipped); false when the
    // offsets end before b (inconsistent with the block count).
    auto seek = [&](std::uint32_t b) {
        for (;;) {
            const unsigned cnt = static_cast<unsigned>(__popcll(__ballot(ends <= b)));
            if (cnt < kWave) {
                w = cbase + cnt;
                we = lane_u32(ends, cnt);
                ws = cnt ? lane_u32(ends, cnt - 1) : cstart;
                return w < a.numWindows;
            }
            cstart = lane_u32(ends, kWave - 1);
            cbase += kWave;
            ends = load_ends();
        }
    };
    if (!seek(u.b0)) return;

    float acc[FT];
#pragma unroll
    for (int f = 0; f < FT; ++f) acc[f] = 0.0f;
    bool touched = false;
    bool open = false;  // blocks of window w accumulated since the last flush

    auto flush = [&]() {
        float s[FT];
#pragma unroll
        for (int f = 0; f < FT; ++f) {
            s[f] = acc[f];
            s[f] += __shfl_xor(s[f], 8);
            s[f] += __shfl_xor(s[f], 16);
            s[f] += __shfl_xor(s[f], 32);
            acc[f] = 0.0f;
        }
        const std::uint64_t tm = __ballot(touched);
        touched = false;
        open = false;
        if (lane < 8) {
            // a phased matrix folds window w into output window w % outWindows,
            // which every phase adds into (atomics into a zeroed Y)
            const std::uint32_t ow = a.outWindows ? w % a.outWindows : w;
            float* o = a.Y + (static_cast<std::uint64_t>(ow) * 8 + j) * a.F;
            if (a.atomicOut || ws < u.b0 || we > u.b1) {  // shared with another unit or phase
                if ((tm >> j) & 0x0101010101010101ull) {
#pragma unroll
                    for (int f = 0; f < FT; ++f)
                        if (static_cast<std::uint32_t>(f) < a.F) atomic_add_f32(o + f, s[f]);
                }
            } else {
#pragma unroll
                for (int f = 0; f < FT; ++f)
                    if (static_cast<std::uint32_t>(f) < a.F) o[f] = a.accumulate ? o[f] + s[f] : s[f];
            }
        }
    };

    NarrowMeta m0 = narrow_meta<VALUES>(a, u.b0, u.b1);
    NarrowMeta m1 = narrow_meta<VALUES>(a, u.b0 + 8, u.b1);
    float x0[FT];
    narrow_row<FT, MODE>(a, m0.in, vec, x0);
    for (std::uint32_t g = u.b0; g < u.b1; g += 8) {
        const NarrowMeta m2 = narrow_meta<VALUES>(a, g + 16, u.b1);
        float x1[FT];
        narrow_row<FT, MODE>(a, m1.in, vec, x1);

        // Output row j of block g+slot.
        const std::uint64_t raw = (static_cast<std::uint64_t>(m0.bitsHi) << 32) | m0.bitsLo;
        const std::uint64_t bm = (MODE == Src::Transposed) ? transpose8x8(raw) : raw;
        const std::uint32_t rb = static_cast<std::uint32_t>(bm >> (8 * j)) & 0xFFu;
        float wv[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            wv[c] = 0.0f;
            if constexpr (VALUES) {
                if ((rb >> c) & 1u) {
                    const unsigned stored = (MODE == Src::Transposed) ? (c * 8 + j) : (j * 8 + c);
                    const unsigned rank = static_cast<unsigned>(__popcll(raw & ((1ull << stored) - 1ull)));
                    wv[c] = a.data[m0.off + rank];
                }
            }
        }
        float x[FT];
#pragma unroll
        for (int f = 0; f < FT; ++f) x[f] = (MODE == Src::Transposed) ? x0[f] : tf32_rna(x0[f]);
        if constexpr (VALUES && MODE != Src::Transposed) {
#pragma unroll
            for (int c = 0; c < 8; ++c) wv[c] = tf32_rna(wv[c]);
        }
        float p[FT];
#pragma unroll
        for (int f = 0; f < FT; ++f) p[f] = 0.0f;
        narrow_columns<0, FT, VALUES>(x, rb, wv, p);

        // Hand the 8 blocks to their windows (usually one).
        const std::uint32_t n = min(8u, u.b1 - g);
        std::uint32_t kk = 0;
        for (;;) {
            const std::uint32_t kend = min(n, we - g);
            if (kend > kk) {
                open = true;
                if (slot >= kk && slot < kend) {
#pragma unroll
                    for (int f = 0; f < FT; ++f) acc[f] += p[f];
                    touched |= rb != 0;
                }
            }
            if (we > g + n) break;  // window w continues past this group
            flush();
            if (g + kend >= u.b1) break;  // the unit ends with window w
            if (!seek(g + kend)) return;
            kk = kend;
            if (kk >= n) break;
        }
        m0 = m1;
        m1 = m2;
#pragma unroll
        for (int f = 0; f < FT; ++f) x0[f] = x1[f];
    }
    if (open) flush();
}

// A grid-stride 16-byte copy (tcc_calibration_copy).
__global__ void calibration_copy_kernel(vu4* __restrict__ dst, const vu4* __restrict__ src, std::uint64_t n) {
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    for (std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = load_global<vu4>(src + i);
}

// Wave w adds 1.0 to the 64 floats of segment w % (rowFloats / 64) of row
// hash(w) % rows, one per lane (tcc_calibration_atomic).
__global__ void calibration_atomic_kernel(float* __restrict__ dst, std::uint32_t rows, std::uint32_t rowFloats,
                                          std::uint64_t waves) {
    const std::uint64_t w = (static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x) / kWave;
    if (w >= waves) return;
    std::uint64_t h = w * 0x9E3779B97F4A7C15ull;  // a multiplicative hash spreads the rows
    h ^= h >> 29;
    const std::uint32_t row = static_cast<std::uint32_t>(h % rows);
    const std::uint32_t seg = static_cast<std::uint32_t>(w % (rowFloats / kWave));
    atomic_add_f32(dst + static_cast<std::uint64_t>(row) * rowFloats + seg * kWave + __lane_id(), 1.0f);
}

// One thread per 4 consecutive features of a row (they lie in one chunk):
// one 8-byte store of their high halves and one 2-byte store of the low bits
// of their two pairs (features past F: the high halves and pair bytes of the
// valid ones only, as the layout's padding is left as it is).  With
// colScale, row r is packed as TF32(colScale[r] * X[r]) (the fp32 product,
// then rounded).  This is thread i's quad: row r, features 4 (i - r quads)
// and on; with smax, the quad's largest finite magnitude goes into its
// slice's LDS maximum.
__device__ __forceinline__ void pack_quad_body(const float* __restrict__ X, std::uint32_t F, std::uint32_t quads,
                                               unsigned char* __restrict__ out, std::uint64_t stride, bool vec2,
                                               const float* __restrict__ colScale, std::uint32_t* smax,
                                               std::uint32_t W, std::uint64_t i, std::uint64_t r) {
    const std::uint32_t e = 4 * static_cast<std::uint32_t>(i - r * quads);
    const std::uint32_t valid = min(4u, F - e);
    const float* x = X + r * F + e;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (vec2 && valid == 4) {
        const vf2 a = load_global<vf2>(x), b = load_global<vf2>(x + 2);
        v[0] = a.x; v[1] = a.y; v[2] = b.x; v[3] = b.y;
    } else {
#pragma unroll
        for (unsigned k = 0; k < 4; ++k)
            if (k < valid) v[k] = x[k];
    }
    if (colScale) {
        const float s = colScale[r];
#pragma unroll
        for (unsigned k = 0; k < 4; ++k) v[k] *= s;
    }
    // A NaN keeps its top 19 bits with the quiet bit set, so that a payload
    // held only in the dropped low bits does not unpack as inf.
    std::uint32_t b[4];
#pragma unroll
    for (unsigned k = 0; k < 4; ++k) {
        const std::uint32_t t = __float_as_uint(tf32_rna(v[k]));
        b[k] = k < valid ? (__builtin_isnan(v[k]) ? (t | 0x00400000u) : t) : 0u;
    }
    if (smax) {
        std::uint32_t m = 0;
#pragma unroll
        for (unsigned k = 0; k < 4; ++k)
            if ((b[k] & 0x7FFFFFFFu) < 0x7F800000u) m = max(m, b[k] & 0x7FFFFFFFu);
        if (m) atomicMax(&smax[e / W], m);
    }
    const auto lo_byte = [](std::uint32_t b0, std::uint32_t b1) {
        return static_cast<unsigned char>(((b0 >> 13) & 7u) | (((b1 >> 13) & 7u) << 3));
    };
    unsigned char* row = out + r * stride;
    const PackedAt at = packed_at(F, e);  // e % 4 == 0: 8-byte aligned high halves, 2-byte aligned pair bytes
    if (valid == 4) {
        *reinterpret_cast<vu2*>(row + at.hi) = vu2{(b[0] >> 16) | (b[1] & 0xFFFF0000u), (b[2] >> 16) | (b[3] & 0xFFFF0000u)};
        *reinterpret_cast<std::uint16_t*>(row + at.lo) =
            static_cast<std::uint16_t>(lo_byte(b[0], b[1]) | (lo_byte(b[2], b[3]) << 8));
    } else {
        for (unsigned k = 0; k < valid; ++k)
            *reinterpret_cast<std::uint16_t*>(row + at.hi + 2 * k) = static_cast<std::uint16_t>(b[k] >> 16);
        row[at.lo] = lo_byte(b[0], b[1]);
        if (valid > 2) row[at.lo + 1] = lo_byte(b[2], b[3]);
    }
}

// With sliceMax (non-null, zeroed by the caller), the largest finite |TF32
// value| bits of each slice of W features (W % 4 == 0) over all rows go to
// sliceMax[(blockIdx.x % kPackSliceMaxRows) * slices + s] through atomicMax:
// each workgroup gathers its own in LDS first.
__global__ void tf32_pack_kernel(const float* __restrict__ X, std::uint32_t rows, std::uint32_t F,
                                 std::uint32_t quads, unsigned char* __restrict__ out, std::uint64_t stride,
                                 bool vec2, const float* __restrict__ colScale, std::uint32_t* __restrict__ sliceMax,
                                 std::uint32_t W, std::uint32_t slices) {
    extern __shared__ std::uint32_t smax[];
    if (sliceMax) {  // uniform
        for (std::uint32_t s = threadIdx.x; s < slices; s += blockDim.x) smax[s] = 0;
        __syncthreads();
    }
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::uint64_t r = i / quads;
    if (r < rows) pack_quad_body(X, F, quads, out, stride, vec2, colScale, sliceMax ? smax : nullptr, W, i, r);
    if (sliceMax) {
        __syncthreads();
        for (std::uint32_t s = threadIdx.x; s < slices; s += blockDim.x)
            if (smax[s]) atomicMax(&sliceMax[(blockIdx.x % kPackSliceMaxRows) * slices + s], smax[s]);
    }
}

struct ScatterArgs {
    const std::uint32_t* winOffset;
    const std::uint32_t* tcOffset;
    const std::uint32_t* idx;  // output rows
    const std::uint64_t* bits;
    const float* data;
    const float* X;
    float* Y;
    std::uint32_t numWindows;
    std::uint32_t numBlocks;
    std::uint32_t numRows;
    std::uint32_t numCols;
    std::uint32_t F;
    std::uint32_t numChunks;
    std::uint32_t unitBlocks;
    std::uint32_t numUnits;
    MixedArgs mixed;
};

// The source columns of a column window that blocks [lo, hi) use: the OR
// over those blocks of their bitmaps' row bytes (one vector load per 64
// blocks, 8 ballots).
__device__ __forceinline__ std::uint32_t used_columns(const std::uint64_t* bits, std::uint32_t lo, std::uint32_t hi) {
    std::uint32_t mask = 0;
    for (std::uint32_t base = lo; base < hi && mask != 0xFFu; base += kWave) {
        const std::uint32_t b = base + __lane_id();
        std::uint32_t cols = 0;
        if (b < hi) {
            std::uint64_t bm = bits[b];
            bm |= bm >> 32;
            bm |= bm >> 16;
            bm |= bm >> 8;
            cols = static_cast<std::uint32_t>(bm) & 0xFFu;
        }
#pragma unroll
        for (int c = 0; c < 8; ++c)
            if (__ballot((cols >> c) & 1u)) mask |= 1u << c;
    }
    return mask;
}

// Row pointers of window w's 8 source columns, resolved lane-parallel: lane
// c < 8 holds column c's (null where `used` omits the column, past numCols
// or without a row).  Resolving column by column put each lookup behind the
// previous column's row load (loads complete in order), one host-link round
// trip per column for the first layer's cold rows.
template <bool MIXED>
__device__ __forceinline__ std::uint64_t window_row_ptrs(const ScatterArgs& a, std::uint32_t w, std::uint32_t used) {
    const unsigned lane = __lane_id();
    const float* row = nullptr;
    const std::uint32_t col = w * 8 + lane;
    if (lane < 8 && ((used >> lane) & 1u) && col < a.numCols) {
        if constexpr (MIXED) {
            // spmm_kernel.cu:521-595: the window's sources resolved once each.
            row = mixed_row(a.mixed, a.F, col);
        } else {
            row = a.X + static_cast<std::uint64_t>(col) * a.F;
        }
    }
    return reinterpret_cast<std::uint64_t>(row);
}

// The window's source rows x[c] from window_row_ptrs (zeros for null), all
// 8 loads issued before any is used; TF32-rounded unless packed as TF32.
// Skipping unused rows matters most for the first layer's cold rows, which
// cross the host link.
template <int V, bool PACKED>
__device__ __forceinline__ void load_window_rows(const ScatterArgs& a, std::uint64_t rowPtrs, std::uint32_t laneOff,
                                                 float (&x)[8][V]) {
    const std::uint32_t lo = static_cast<std::uint32_t>(rowPtrs);
    const std::uint32_t hi = static_cast<std::uint32_t>(rowPtrs >> 32);
    if constexpr (PACKED) {  // packed TF32 feature rows: no rounding needed
        const std::uint32_t records = rowPtrs ? ~0u : 0u;  // the buffer bound of this lane's row
        PackedVec<V> pk[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const std::uint64_t rp = (static_cast<std::uint64_t>(lane_u32(hi, c)) << 32) | lane_u32(lo, c);
            pk[c] = load_packed<V>(rp, lane_u32(records, c), a.F, laneOff);
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) unpack<V>(pk[c], x[c]);
        return;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const std::uint64_t rp = (static_cast<std::uint64_t>(lane_u32(hi, c)) << 32) | lane_u32(lo, c);
#pragma unroll
        for (int v = 0; v < V; ++v) x[c][v] = 0.0f;
        if (rp != 0) {
            const Vec<V> t = load_vec<V>(reinterpret_cast<const float*>(rp) + laneOff);
#pragma unroll
            for (int v = 0; v < V; ++v) x[c][v] = t.v[v];
        }
    }
#pragma unroll
    for (int c = 0; c < 8; ++c)
#pragma unroll
        for (int v = 0; v < V; ++v) x[c][v] = tf32_rna(x[c][v]);
}

// Block b's metadata as one word per lane, read with v_readlane when the
// block is processed: lanes 0-7 the output rows of its 8 block rows, lanes
// 8-9 its bitmap and, with values, lanes 10-11 block b+1's bitmap and lane
// 12 block b+1's value offset (so that b+1's values can be loaded while b
// is processed).  Loaded one block ahead, before the block's atomics: loads
// and atomics complete in order, so a load issued after them and used at
// once would wait for all of them.
template <bool VALUES>
__device__ __forceinline__ std::uint32_t scatter_meta(const ScatterArgs& a, std::uint32_t b) {
    const unsigned lane = __lane_id();
    const std::uint32_t* bitsw = reinterpret_cast<const std::uint32_t*>(a.bits);
    std::uint32_t m = 0;
    if (lane < 8) {
        m = a.idx[static_cast<std::uint64_t>(b) * 8 + lane];
    } else if (lane < 10) {
        m = bitsw[2ull * b + (lane - 8)];
    } else if (VALUES && b + 1 < a.numBlocks) {
        if (lane < 12) m = bitsw[2ull * (b + 1) + (lane - 10)];
        else if (lane == 12) m = a.tcOffset[b + 1];
    }
    return m;
}

__device__ __forceinline__ std::uint64_t meta_bits(std::uint32_t m, int lane0) {
    return (static_cast<std::uint64_t>(lane_u32(m, lane0 + 1)) << 32) | lane_u32(m, lane0);
}

// Lane i: the value of the i-th stored nonzero of a block with bitmap `bits`
// whose values start at data[off] (unrounded; zero past its count).
__device__ __forceinline__ float scatter_vals(const ScatterArgs& a, std::uint64_t bits, std::uint32_t off) {
    return __lane_id() < static_cast<unsigned>(__popcll(bits)) ? a.data[off + __lane_id()] : 0.0f;
}

template <int V, bool MIXED, bool VALUES, bool PACKED = false>
__device__ __forceinline__ void scatter_body(const ScatterArgs& a, std::uint32_t gw) {
    const unsigned lane = __lane_id();
    const std::uint32_t chunk = gw / a.numUnits;
    const std::uint32_t unit = gw - chunk * a.numUnits;
    if (chunk >= a.numChunks) return;
    const UnitRange u = unit_range(a.winOffset, a.numWindows, a.numBlocks, a.unitBlocks, a.numUnits, unit);
    if (u.b0 >= u.b1 || u.w >= a.numWindows) return;
    const std::uint32_t f0 = chunk * (kWave * V) + lane * V;
    const bool active = f0 < a.F;
    const std::uint32_t laneOff = active ? f0 : f0 - lane * V;  // inactive: lane 0's features

    std::uint32_t w = u.w;
    std::uint32_t we = a.winOffset[w + 1];
    while (we <= u.b0 && w + 1 < a.numWindows) {  // skip empty windows starting at b0
        ++w;
        we = a.winOffset[w + 1];
    }
    float x[8][V];
    load_window_rows<V, PACKED>(a, window_row_ptrs<MIXED>(a, w, used_columns(a.bits, u.b0, min(we, u.b1))), laneOff,
                                x);
    std::uint32_t cur = scatter_meta<VALUES>(a, u.b0);
    float curVals = 0.0f;
    if constexpr (VALUES) curVals = scatter_vals(a, a.bits[u.b0], a.tcOffset[u.b0]);
    for (std::uint32_t b = u.b0; b < u.b1; ++b) {
        if (b >= we) {
            do {
                ++w;
                we = a.winOffset[w + 1];
            } while (b >= we && w + 1 < a.numWindows);
            load_window_rows<V, PACKED>(a, window_row_ptrs<MIXED>(a, w, used_columns(a.bits, b, min(we, u.b1))), laneOff,
                                        x);
        }
        const std::uint64_t bm = meta_bits(cur, 8);
        // the next block's metadata and values, loaded before this block's atomics
        std::uint32_t nxt = cur;
        float nxtVals = curVals;
        if (b + 1 < u.b1) {
            nxt = scatter_meta<VALUES>(a, b + 1);
            if constexpr (VALUES) nxtVals = scatter_vals(a, meta_bits(cur, 10), lane_u32(cur, 12));
        }
        float vals = 0.0f;
        if constexpr (VALUES) vals = tf32_rna(curVals);
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const std::uint32_t rb = static_cast<std::uint32_t>(bm >> (8 * r)) & 0xFFu;
            if (rb == 0) continue;
            const std::uint32_t row = lane_u32(cur, r);
            if (row >= a.numRows) continue;  // spmm_kernel.cu:2025-2044
            float s[V];
#pragma unroll
            for (int v = 0; v < V; ++v) s[v] = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                if (!(rb & (1u << c))) continue;
                if constexpr (VALUES) {
                    const int rank = static_cast<int>(__popcll(bm & ((1ull << (r * 8 + c)) - 1ull)));
                    const float wv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(vals), rank));
#pragma unroll
                    for (int v = 0; v < V; ++v) s[v] = fmaf(wv, x[c][v], s[v]);
                } else {
#pragma unroll
                    for (int v = 0; v < V; ++v) s[v] += x[c][v];
                }
            }
            if (active) {
                float* out = a.Y + static_cast<std::uint64_t>(row) * a.F + f0;
#pragma unroll
                for (int v = 0; v < V; ++v)
                    if (f0 + v < a.F) atomic_add_f32(out + v, s[v]);
            }
        }
        cur = nxt;
        curVals = nxtVals;
    }
}

template <int V, bool MIXED, bool VALUES>
__global__ void __launch_bounds__(kThreads) scatter_kernel(ScatterArgs a) {
    scatter_body<V, MIXED, VALUES>(a, blockIdx.x * kWaves + uniform(threadIdx.x / kWave));
}

// The first layer's forward in one launch.  The reference runs the hot BCSR
// gather and the cold BCSC scatter one after the other
// (spmm_launcher.cu:30-271); here they run side by side.  `scatterWGs`
// persistent scatter workgroups walk the scatter's (unit, chunk) waves with
// a grid stride, so that a fixed number of waves keeps the host link busy
// for the whole launch; the other workgroups are the gather's, streaming
// HBM.  Workgroups are dispatched to the 8 XCDs round-robin, so the scatter
// takes the workgroups i < 8*perXcd with i % 8 < xcds: it runs on `xcds`
// XCDs of its own, apart from the gather's memory traffic (the two slowed
// each other down when they shared compute units).  The placement only
// affects speed: every scatter workgroup index is launched.  Both parts add
// into a zeroed Y with atomics.
template <int V, bool GVALUES, bool SVALUES, bool PACKED>
__global__ void __launch_bounds__(kThreads) mixed_forward_kernel(GatherArgs g, ScatterArgs s, std::uint32_t xcds,
                                                                 std::uint32_t perXcd) {
    const std::uint32_t i = blockIdx.x;
    const std::uint32_t wave = uniform(threadIdx.x / kWave);
    const std::uint32_t slot = i & 7u;
    const bool head = i < 8u * perXcd;
    if (head && slot < xcds) {
        const std::uint32_t scatterWGs = xcds * perXcd;
        const std::uint64_t waves = static_cast<std::uint64_t>(s.numUnits) * s.numChunks;
        for (std::uint64_t gw = static_cast<std::uint64_t>((i >> 3) * xcds + slot) * kWaves + wave; gw < waves;
             gw += static_cast<std::uint64_t>(scatterWGs) * kWaves)
            scatter_body<V, true, SVALUES, PACKED>(s, static_cast<std::uint32_t>(gw));
    } else if (g.numUnits != 0) {  // no gather units: no row windows
        // scatter workgroups before i
        const std::uint32_t before = head ? (i >> 3) * xcds + min(slot, xcds) : xcds * perXcd;
        gather_body<V, PACKED ? Src::MixedPacked : Src::Mixed, GVALUES>(g, (i - before) * kWaves + wave);
    }
}

// Vector width per lane: the narrowest V in {1,2,4} whose 64*V-feature chunk
// covers F (so a wave's lanes are all busy), else the widest that divides F;
// V-wide loads need F % V == 0 and 4V-byte aligned base pointers.
inline int pick_vec(std::uint32_t F, std::initializer_list<const void*> ptrs) {
    auto ok = [&](int V) {
        if (F % V != 0) return false;
        for (const void* p : ptrs)
            if (p && (reinterpret_cast<std::uintptr_t>(p) % (4u * V)) != 0) return false;
        return true;
    };
    for (int V : {1, 2, 4})
        if (64u * V >= F && ok(V)) return V;
    for (int V : {4, 2})
        if (ok(V)) return V;
    return 1;
}

// Blocks per unit: `requested` if nonzero, else about one wave of work per
// wave slot of the device (32 per CU), a power of two in [16, maxK]: fewer,
// longer units pay the per-wave start (window search, first metadata group)
// less often.  Gathers from device rows cap units at 128 blocks: past that
// the waves in flight spread over more of the rows (config 3: 21.3 ms with
// 1024-block units, 20.0 ms with 128).  The first-layer forward, whose cold
// rows come over the host link, and the scatters keep 1024 (config 4:
// 9.1 ms, against 10.4 ms with 128).
constexpr std::uint32_t kDeviceRowsMaxUnit = 128;
constexpr std::uint32_t kHostLinkMaxUnit = 1024;

inline std::uint32_t unit_blocks(std::uint32_t requested, std::uint32_t blocks, std::uint32_t chunks,
                                 std::uint32_t maxK) {
    if (requested != 0) return requested;
    const std::uint64_t work = static_cast<std::uint64_t>(blocks) * chunks;
    const std::uint64_t slots = static_cast<std::uint64_t>(device_cus()) * 32;
    std::uint32_t K = 16;
    while (K < maxK && static_cast<std::uint64_t>(K) * slots < work) K *= 2;
    return K;
}

// Work split of a gather (chunks, unit size, units); its wave count.
inline std::uint64_t plan_gather(GatherArgs& a, int V, std::uint32_t requestedK,
                                 std::uint32_t maxK = kDeviceRowsMaxUnit) {
    if (a.numWindows == 0) return 0;
    const std::uint32_t features = (a.featureEnd ? a.featureEnd : a.F) - a.featureBase;
    a.numChunks = (features + kWave * V - 1) / (kWave * V);
    a.unitBlocks = unit_blocks(requestedK, a.numBlocks, a.numChunks, maxK);
    a.numUnits = std::max<std::uint32_t>(1, (a.numBlocks + a.unitBlocks - 1) / a.unitBlocks);
    return static_cast<std::uint64_t>(a.numUnits) * a.numChunks;
}

// Work split of a scatter; its wave count.
inline std::uint64_t plan_scatter(ScatterArgs& a, int V, std::uint32_t requestedK) {
    if (a.numWindows == 0 || a.numBlocks == 0) return 0;
    a.numChunks = (a.F + kWave * V - 1) / (kWave * V);
    a.unitBlocks = unit_blocks(requestedK, a.numBlocks, a.numChunks, kHostLinkMaxUnit);
    a.numUnits = (a.numBlocks + a.unitBlocks - 1) / a.unitBlocks;
    return static_cast<std::uint64_t>(a.numUnits) * a.numChunks;
}

// Zeroes, over all F features, the windows that several units of a planned
// gather add into (none when one unit covers each window, or when the gather
// adds into Y or writes through atomics).
int zero_shared(const GatherArgs& a, hipStream_t st) {
    if (a.numWindows == 0 || a.numUnits <= 1 || a.accumulate || a.atomicOut) return TCC_OK;
    hipLaunchKernelGGL(zero_shared_windows_kernel, dim3(grid_for(a.numWindows, kThreads)), dim3(kThreads), 0, st,
                       a.winOffset, a.numWindows, a.unitBlocks, a.Y, a.F);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

// zeroShared = false: a launch over other features of units whose shared
// windows were zeroed already.
template <Src MODE>
int launch_gather(GatherArgs a, int V, std::uint32_t requestedK, hipStream_t st, bool zeroShared = true) {
    constexpr bool kHostRows = MODE == Src::Mixed || MODE == Src::MixedPacked;
    const std::uint64_t waves = plan_gather(a, V, requestedK, kHostRows ? kHostLinkMaxUnit : kDeviceRowsMaxUnit);
    if (waves == 0) return TCC_OK;
    TCC_REQUIRE(waves <= 0xFFFFFFFFull / kWaves, TCC_ERR_UNSUPPORTED, "SpMM launch too large");
    if (zeroShared) {
        const int rc = zero_shared(a, st);
        if (rc) return rc;
    }
    const dim3 grid(grid_for(waves, kWaves));
    if (a.data != nullptr) {
        if (V == 4) hipLaunchKernelGGL((gather_kernel<4, MODE, true>), grid, dim3(kThreads), 0, st, a);
        else if (V == 2) hipLaunchKernelGGL((gather_kernel<2, MODE, true>), grid, dim3(kThreads), 0, st, a);
        else hipLaunchKernelGGL((gather_kernel<1, MODE, true>), grid, dim3(kThreads), 0, st, a);
    } else {
        if (V == 4) hipLaunchKernelGGL((gather_kernel<4, MODE, false>), grid, dim3(kThreads), 0, st, a);
        else if (V == 2) hipLaunchKernelGGL((gather_kernel<2, MODE, false>), grid, dim3(kThreads), 0, st, a);
        else hipLaunchKernelGGL((gather_kernel<1, MODE, false>), grid, dim3(kThreads), 0, st, a);
    }
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

// Feature widths the narrow gather takes (one wave per 8 blocks).
constexpr std::uint32_t kNarrowMaxF = 16;
// Mean gathers per input row from which packing X to TF32 rows pays off.
constexpr std::uint64_t kPackMinGathers = 16;

// Blocks per unit of the narrow gather: `requested` if nonzero, else about
// four units per wave slot (a unit's 8-block steps are short, so waves are
// plentiful), a power of two in [64, 4096].
inline std::uint32_t narrow_unit_blocks(std::uint32_t requested, std::uint32_t blocks) {
    if (requested != 0) return requested;
    const std::uint64_t units = static_cast<std::uint64_t>(device_cus()) * 32 * 4;
    std::uint32_t K = 64;
    while (K < 4096 && static_cast<std::uint64_t>(K) * units < blocks) K *= 2;
    return K;
}

template <int FT, Src MODE>
void narrow_dispatch(const GatherArgs& a, dim3 grid, hipStream_t st) {
    if (a.data != nullptr) hipLaunchKernelGGL((narrow_gather_kernel<FT, MODE, true>), grid, dim3(kThreads), 0, st, a);
    else hipLaunchKernelGGL((narrow_gather_kernel<FT, MODE, false>), grid, dim3(kThreads), 0, st, a);
}

template <Src MODE>
int launch_narrow(GatherArgs a, std::uint32_t requestedK, hipStream_t st) {
    static_assert(MODE == Src::Plain || MODE == Src::Transposed, "narrow gather reads X or dY");
    if (a.numWindows == 0) return TCC_OK;
    const std::uint64_t outWindows = a.outWindows ? a.outWindows : a.numWindows;
    if (!a.accumulate) TCC_HIP_CHECK(fill<float>(a.Y, outWindows * 8 * a.F, 0.0f, st));
    if (a.numBlocks == 0) return TCC_OK;
    a.numChunks = 1;
    a.unitBlocks = narrow_unit_blocks(requestedK, a.numBlocks);
    a.numUnits = (a.numBlocks + a.unitBlocks - 1) / a.unitBlocks;
    const dim3 grid(grid_for(a.numUnits, kWaves));
    if (a.F <= 2) narrow_dispatch<2, MODE>(a, grid, st);
    else if (a.F <= 4) narrow_dispatch<4, MODE>(a, grid, st);
    else if (a.F <= 8) narrow_dispatch<8, MODE>(a, grid, st);
    else narrow_dispatch<16, MODE>(a, grid, st);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

template <bool MIXED>
int launch_scatter(ScatterArgs a, int V, std::uint32_t requestedK, hipStream_t st) {
    const std::uint64_t waves = plan_scatter(a, V, requestedK);
    if (waves == 0) return TCC_OK;
    TCC_REQUIRE(waves <= 0xFFFFFFFFull / kWaves, TCC_ERR_UNSUPPORTED, "SpMM launch too large");
    const dim3 grid(grid_for(waves, kWaves));
    if (a.data != nullptr) {
        if (V == 4) hipLaunchKernelGGL((scatter_kernel<4, MIXED, true>), grid, dim3(kThreads), 0, st, a);
        else if (V == 2) hipLaunchKernelGGL((scatter_kernel<2, MIXED, true>), grid, dim3(kThreads), 0, st, a);
        else hipLaunchKernelGGL((scatter_kernel<1, MIXED, true>), grid, dim3(kThreads), 0, st, a);
    } else {
        if (V == 4) hipLaunchKernelGGL((scatter_kernel<4, MIXED, false>), grid, dim3(kThreads), 0, st, a);
        else if (V == 2) hipLaunchKernelGGL((scatter_kernel<2, MIXED, false>), grid, dim3(kThreads), 0, st, a);
        else hipLaunchKernelGGL((scatter_kernel<1, MIXED, false>), grid, dim3(kThreads), 0, st, a);
    }
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

MixedArgs mixed_args(const tcc_feature_source* src, std::uint32_t F) {
    MixedArgs m{};
    m.rowBytes = src->row_format == TCC_ROWS_TF32_PACKED ? packed_stride(F) : 0;
    m.idMap = src->id_map;
    m.cacheSearchMap = src->cache_search_map;
    m.gpuCache = src->gpu_feature_cache;
    m.gpuNodeCapacity = src->gpu_node_capacity;
    m.cpuFeatures = src->cpu_features;
    m.cpuLen = src->cpu_feature_len;
    m.gpuCacheCount = src->gpu_feature_cache_count;
    m.deviceError = src->device_error;
    return m;
}

GatherArgs bcsr_args(const tcc_bcsr* A, const float* X, float* Y, std::uint32_t F, int accumulate) {
    GatherArgs a{};
    a.winOffset = A->rowWindowOffset;
    a.tcOffset = A->tcOffset;
    a.idx = A->sparseA2B;
    a.bits = A->tcLocalBit;
    a.data = A->data;
    a.X = X;
    a.Y = Y;
    a.numWindows = A->num_rowWindows;
    a.numBlocks = A->num_TCBlocks;
    a.numIn = A->num_cols;
    a.F = F;
    a.accumulate = accumulate;
    if (A->phases > 1) {  // phased: every window adds into window w % outWindows
        a.outWindows = A->num_rowWindows / A->phases;
        a.atomicOut = 1;
    }
    return a;
}

// Y of a phased product receives atomics only: zero it first unless adding.
hipError_t zero_phased_output(const GatherArgs& a, hipStream_t st) {
    if (a.outWindows == 0 || a.accumulate) return hipSuccess;
    return fill<float>(a.Y, static_cast<std::uint64_t>(a.outWindows) * 8 * a.F, 0.0f, st);
}

ScatterArgs bcsc_args(const tcc_bcsc* A, const float* X, float* Y, std::uint32_t F) {
    ScatterArgs a{};
    a.winOffset = A->colWindowOffset;
    a.tcOffset = A->tcOffset;
    a.idx = A->sparseA2C;
    a.bits = A->tcLocalBit;
    a.data = A->data;
    a.X = X;
    a.Y = Y;
    a.numWindows = A->num_colWindows;
    a.numBlocks = A->num_TCBlocks;
    a.numRows = A->num_rows;
    a.numCols = A->num_cols;
    a.F = F;
    return a;
}

// Feature source checks: the fields every lookup reads, a known row format,
// and 16-byte aligned host rows for packed tables.
bool source_ok(const tcc_feature_source* src) {
    if (!(src && src->id_map && src->cache_search_map && src->gpu_feature_cache && src->gpu_node_capacity > 0))
        return false;
    if (src->row_format == TCC_ROWS_FP32) return true;
    return src->row_format == TCC_ROWS_TF32_PACKED && reinterpret_cast<std::uintptr_t>(src->cpu_features) % 16 == 0;
}

// Vector width of a first-layer product: packed rows longer than one chunk
// are gathered a chunk at a time (4 features a lane), as tcc_bcsr_spmm_packed.
int mixed_vec(const tcc_feature_source* src, std::uint32_t F, const float* Y) {
    if (src->row_format == TCC_ROWS_TF32_PACKED) return F > kPackChunk ? 4 : pick_vec(F, {Y});
    return pick_vec(F, {Y, src->cpu_features});
}

// The window offsets are read whenever there are windows (a gather writes
// every window, empty or not), the block arrays only when there are blocks:
// a matrix without blocks may come with empty (null) block tensors.
bool bcsr_ok(const tcc_bcsr* A) {
    return A && (A->num_rowWindows == 0 || A->rowWindowOffset) &&
           (A->num_TCBlocks == 0 || (A->rowWindowOffset && A->sparseA2B && A->tcLocalBit)) &&
           (A->data == nullptr || A->tcOffset != nullptr) &&
           (A->phases <= 1 || A->num_rowWindows % A->phases == 0);
}

bool bcsc_ok(const tcc_bcsc* A) {
    return A && (A->num_TCBlocks == 0 || (A->colWindowOffset && A->sparseA2C && A->tcLocalBit)) &&
           (A->data == nullptr || A->tcOffset != nullptr);
}

}  // namespace

// ---------------------------------------------------------------- scaled forms (gather_ops.hpp)

int bcsr_spmm_scaled(const tcc_bcsr* A, const float* X, float* Y, std::uint32_t featureDim, int accumulate,
                     const float* rowScale, hipStream_t st, std::uint32_t rowLimit) {
    TCC_REQUIRE(bcsr_ok(A) && X && Y && feature_dim_ok(featureDim), TCC_ERR_INVALID_ARGUMENT,
                "invalid BCSR SpMM arguments");
    TCC_REQUIRE(rowLimit == 0 || (accumulate && A->phases <= 1 && rowLimit <= 8ull * A->num_rowWindows &&
                                  rowLimit > 8ull * A->num_rowWindows - 8),
                TCC_ERR_INVALID_ARGUMENT,
                "a row limit needs accumulate and an unphased BCSR, and must fall in the last window");
    // the narrow gather has neither row scales nor a row limit: such
    // products take the wide one
    if (featureDim <= kNarrowMaxF && rowScale == nullptr && rowLimit == 0)
        return launch_narrow<Src::Plain>(bcsr_args(A, X, Y, featureDim, accumulate), A->unitBlocks, st);
    GatherArgs a = bcsr_args(A, X, Y, featureDim, accumulate);
    a.rowScale = rowScale;
    a.rowLimit = rowLimit;
    TCC_HIP_CHECK(zero_phased_output(a, st));
    return launch_gather<Src::Plain>(a, pick_vec(featureDim, {X, Y}), A->unitBlocks, st);
}

int tf32_pack_scaled(const float* X, std::uint32_t rows, std::uint32_t featureDim, const float* colScale,
                     void* packed, hipStream_t st, std::uint32_t* sliceMax, std::uint32_t sliceWidth,
                     std::uint32_t slices) {
    TCC_REQUIRE(X && packed && feature_dim_ok(featureDim), TCC_ERR_INVALID_ARGUMENT, "invalid TF32 pack arguments");
    TCC_REQUIRE(reinterpret_cast<std::uintptr_t>(packed) % 16 == 0, TCC_ERR_INVALID_ARGUMENT,
                "packed buffer must be 16-byte aligned");
    if (rows == 0) return TCC_OK;
    const std::uint32_t quads = (featureDim + 3) / 4;
    const std::uint64_t n = static_cast<std::uint64_t>(rows) * quads;
    TCC_REQUIRE(n <= 0xFFFFFFFFull * 256, TCC_ERR_UNSUPPORTED, "TF32 pack too large");
    // two 8-byte loads a thread when every row starts 8-byte aligned
    const bool vec2 = featureDim % 2 == 0 && reinterpret_cast<std::uintptr_t>(X) % 8 == 0;
    if (sliceMax) {
        TCC_REQUIRE(sliceWidth % 4 == 0 && sliceWidth > 0 && slices > 0 && slices <= kPackMaxSlices &&
                        static_cast<std::uint64_t>(slices) * sliceWidth >= featureDim,
                    TCC_ERR_INVALID_ARGUMENT, "invalid slice maxima of the TF32 pack");
        TCC_HIP_CHECK(fill<std::uint32_t>(sliceMax, static_cast<std::uint64_t>(kPackSliceMaxRows) * slices, 0u, st));
    }
    hipLaunchKernelGGL(tf32_pack_kernel, dim3(grid_for(n, 256)), dim3(256),
                       sliceMax ? slices * sizeof(std::uint32_t) : 0, st, X, rows, featureDim, quads,
                       static_cast<unsigned char*>(packed), packed_stride(featureDim), vec2, colScale, sliceMax,
                       sliceWidth, slices);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

// A second stream per device, for work that runs beside a launch on the
// caller's stream (default priority, non-blocking).  SideFork orders it
// after the work queued so far on st (fork) and st after everything queued
// on it in between (join); when st is being captured, belongs to another
// device than the current one, or the side stream cannot be made, the work
// goes to st itself.  The lock keeps concurrent
// callers' record/wait pairs on the shared events apart: a wait takes the
// event's latest record.
namespace {

struct SideLane {
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
std::mutex g_sideMutex;
SideLane g_sideLanes[64];

class SideFork {
public:
    explicit SideFork(hipStream_t st) : st_(st) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(st, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) return;
        // the side stream is made on the current device: st must be one of its streams
        int dev = 0;
        hipDevice_t stDev = -1;
        if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || hipStreamGetDevice(st, &stDev) != hipSuccess ||
            stDev != dev)
            return;
        lock_ = std::unique_lock<std::mutex>(g_sideMutex);
        SideLane& l = g_sideLanes[dev];
        if (!l.stream) {
            hipStream_t s = nullptr;
            hipEvent_t f = nullptr, j = nullptr;
            if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return;
            if (hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
                hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
                if (f) (void)hipEventDestroy(f);
                (void)hipStreamDestroy(s);
                return;
            }
            l.stream = s;
            l.fork = f;
            l.join = j;
        }
        if (hipEventRecord(l.fork, st) != hipSuccess || hipStreamWaitEvent(l.stream, l.fork, 0) != hipSuccess) return;
        lane_ = &l;
    }
    SideFork(const SideFork&) = delete;
    SideFork& operator=(const SideFork&) = delete;
    ~SideFork() { (void)join(); }

    hipStream_t stream() const { return lane_ ? lane_->stream : st_; }

    // Orders st after the side stream's work; idempotent.
    int join() {
        if (!lane_) return TCC_OK;
        SideLane* l = lane_;
        lane_ = nullptr;
        TCC_HIP_CHECK(hipEventRecord(l->join, l->stream));
        TCC_HIP_CHECK(hipStreamWaitEvent(st_, l->join, 0));
        return TCC_OK;
    }

private:
    hipStream_t st_;
    SideLane* lane_ = nullptr;
    std::unique_lock<std::mutex> lock_;
};

}  // namespace

int bcsr_spmm_packed_scaled(const tcc_bcsr* A, const void* packedX, float* Y, std::uint32_t featureDim,
                            int accumulate, const float* rowScale, hipStream_t st, std::uint32_t rowLimit) {
    TCC_REQUIRE(bcsr_ok(A) && packedX && Y && feature_dim_ok(featureDim), TCC_ERR_INVALID_ARGUMENT,
                "invalid packed BCSR SpMM arguments");
    TCC_REQUIRE(rowLimit == 0 || (accumulate && A->phases <= 1 && rowLimit <= 8ull * A->num_rowWindows &&
                                  rowLimit > 8ull * A->num_rowWindows - 8),
                TCC_ERR_INVALID_ARGUMENT,
                "a row limit needs accumulate and an unphased BCSR, and must fall in the last window");
    TCC_REQUIRE(reinterpret_cast<std::uintptr_t>(packedX) % 16 == 0, TCC_ERR_INVALID_ARGUMENT,
                "packed buffer must be 16-byte aligned");
    GatherArgs a = bcsr_args(A, nullptr, Y, featureDim, accumulate);
    a.rowScale = rowScale;
    a.rowLimit = rowLimit;
    TCC_HIP_CHECK(zero_phased_output(a, st));
    a.packed = static_cast<const unsigned char*>(packedX);
    a.packedStride = static_cast<std::uint32_t>(packed_stride(featureDim));
    // Rows longer than one chunk are gathered a whole chunk (4 features a
    // lane) at a time, whatever F % 4, so that each load covers its lines.
    if (featureDim <= kPackChunk) return launch_gather<Src::Packed>(a, pick_vec(featureDim, {Y}), A->unitBlocks, st);
    // A last chunk of at most 128 features would leave most lanes of its
    // 4-wide waves idle while costing as much as a full chunk (each block is
    // one memory round trip either way): its waves run on their own, 2 or 1
    // features a lane, over the same units, after the full chunks.
    const std::uint32_t tail = featureDim % kPackChunk;
    if (tail == 0 || tail > kPackChunk / 2) return launch_gather<Src::Packed>(a, 4, A->unitBlocks, st);
    // Both launches take the full chunks' units, whose shared windows are
    // zeroed (over all F) before either starts.  The last chunk runs on the
    // device's side stream beside the full chunks, so that its waves fill
    // the CUs the full launch's last waves leave idle (on a stream being
    // captured, after them on st).
    GatherArgs full = a;
    full.featureEnd = featureDim - tail;
    GatherArgs last = a;
    last.featureBase = featureDim - tail;
    if (plan_gather(full, 4, A->unitBlocks) == 0) return TCC_OK;
    int rc = zero_shared(full, st);
    if (rc) return rc;
    const int lastV = tail > kWave ? 2 : 1;
    SideFork side(st);
    rc = launch_gather<Src::Packed>(last, lastV, full.unitBlocks, side.stream(), false);
    if (rc == TCC_OK) rc = launch_gather<Src::Packed>(full, 4, A->unitBlocks, st, false);
    const int joined = side.join();
    return rc ? rc : joined;
}

}  // namespace tcc

using namespace tcc;

extern "C" {

int tcc_bcsr_spmm(const tcc_bcsr* A, const float* X, float* Y, std::uint32_t featureDim, int accumulate,
                  void* stream) {
    clear_last_error();
    return bcsr_spmm_scaled(A, X, Y, featureDim, accumulate, nullptr, as_stream(stream));
}

size_t tcc_tf32_packed_bytes(std::uint32_t rows, std::uint32_t featureDim) {
    return static_cast<size_t>(rows) * packed_stride(featureDim);
}

int tcc_calibration_copy(void* dst, const void* src, size_t bytes, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bytes % 16 == 0 && (bytes == 0 || (dst && src)) && reinterpret_cast<std::uintptr_t>(dst) % 16 == 0 &&
                    reinterpret_cast<std::uintptr_t>(src) % 16 == 0,
                TCC_ERR_INVALID_ARGUMENT, "calibration copy: 16-byte multiples and alignment");
    if (bytes == 0) return TCC_OK;
    const std::uint64_t n = bytes / 16;
    hipLaunchKernelGGL(calibration_copy_kernel, dim3(static_cast<unsigned>(std::min<std::uint64_t>((n + 255) / 256, 65536))),
                       dim3(256), 0, as_stream(stream), static_cast<vu4*>(dst), static_cast<const vu4*>(src), n);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

int tcc_calibration_atomic(float* dst, std::uint32_t rows, std::uint32_t rowFloats, std::uint64_t waves,
                           void* stream) {
    clear_last_error();
    TCC_REQUIRE(dst && rows > 0 && rowFloats >= kWave && rowFloats % kWave == 0, TCC_ERR_INVALID_ARGUMENT,
                "calibration atomic: rows > 0, rowFloats a multiple of 64");
    if (waves == 0) return TCC_OK;
    TCC_REQUIRE(waves <= 0xFFFFFFFFull / kWaves * kWaves, TCC_ERR_UNSUPPORTED, "calibration atomic: too many waves");
    hipLaunchKernelGGL(calibration_atomic_kernel, dim3(grid_for(waves * kWave, kThreads)), dim3(kThreads), 0,
                       as_stream(stream), dst, rows, rowFloats, waves);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

int tcc_tf32_pack(const float* X, std::uint32_t rows, std::uint32_t featureDim, void* packed, void* stream) {
    clear_last_error();
    return tf32_pack_scaled(X, rows, featureDim, nullptr, packed, as_stream(stream));
}

int tcc_bcsr_spmm_packed(const tcc_bcsr* A, const void* packedX, float* Y, std::uint32_t featureDim, int accumulate,
                         void* stream) {
    clear_last_error();
    return bcsr_spmm_packed_scaled(A, packedX, Y, featureDim, accumulate, nullptr, as_stream(stream));
}

int tcc_bcsr_spmm_mixed(const tcc_bcsr* A, const tcc_feature_source* src, float* Y, std::uint32_t featureDim,
                        int accumulate, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsr_ok(A) && source_ok(src) && Y && feature_dim_ok(featureDim), TCC_ERR_INVALID_ARGUMENT,
                "invalid mixed BCSR SpMM arguments");
    TCC_REQUIRE(A->phases <= 1, TCC_ERR_UNSUPPORTED, "the mixed SpMM takes an ordinary (unphased) BCSR");
    GatherArgs a = bcsr_args(A, nullptr, Y, featureDim, accumulate);
    a.mixed = mixed_args(src, featureDim);
    // Hot-cache bases live in a device pointer table and are taken to be
    // 16-byte aligned (hipMalloc / torch allocations); host rows are checked.
    const int V = mixed_vec(src, featureDim, Y);
    if (src->row_format == TCC_ROWS_TF32_PACKED)
        return launch_gather<Src::MixedPacked>(a, V, A->unitBlocks, as_stream(stream));
    return launch_gather<Src::Mixed>(a, V, A->unitBlocks, as_stream(stream));
}

int tcc_bcsc_spmm(const tcc_bcsc* A, const float* X, float* Y, std::uint32_t featureDim, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsc_ok(A) && X && Y && feature_dim_ok(featureDim), TCC_ERR_INVALID_ARGUMENT,
                "invalid BCSC SpMM arguments");
    return launch_scatter<false>(bcsc_args(A, X, Y, featureDim), pick_vec(featureDim, {X, Y}), A->unitBlocks,
                                 as_stream(stream));
}

int tcc_bcsc_transpose_spmm(const tcc_bcsc* A, const float* dY, float* dX, std::uint32_t featureDim,
                            int accumulate, void* stream) {
    clear_last_error();
    // the gather walks every column window (empty ones write zeros): offsets needed
    TCC_REQUIRE(bcsc_ok(A) && (A->num_colWindows == 0 || A->colWindowOffset) && dY && dX &&
                    feature_dim_ok(featureDim),
                TCC_ERR_INVALID_ARGUMENT, "invalid transposed BCSC SpMM arguments");
    GatherArgs a{};
    a.winOffset = A->colWindowOffset;
    a.tcOffset = A->tcOffset;
    a.idx = A->sparseA2C;
    a.bits = A->tcLocalBit;
    a.data = A->data;
    a.X = dY;
    a.Y = dX;
    a.numWindows = A->num_colWindows;
    a.numBlocks = A->num_TCBlocks;
    a.numIn = A->num_rows;
    a.F = featureDim;
    a.accumulate = accumulate;
    if (featureDim <= kNarrowMaxF) return launch_narrow<Src::Transposed>(a, A->unitBlocks, as_stream(stream));
    const int V = pick_vec(featureDim, {dY, dX});
    return launch_gather<Src::Transposed>(a, V, A->unitBlocks, as_stream(stream));
}

int tcc_spmm_cnic_forward(const tcc_bcsr* bcsr, const tcc_bcsc* bcsc, const float* X, float* denseC,
                          std::uint32_t featureDim, void* stream) {
    return tcc_spmm_cnic_forward_ws(bcsr, bcsc, X, denseC, featureDim, nullptr, 0, stream);
}

size_t tcc_spmm_cnic_forward_workspace_bytes(const tcc_bcsr* bcsr, std::uint32_t featureDim) {
    if (!bcsr || featureDim <= kNarrowMaxF || bcsr->num_cols == 0) return 0;
    // rows gathered 16 times on average (8 per block): packing pays
    // (config 3, 441 gathers a row: 36.7 -> 21.5 ms; config 2, 7.3: a loss)
    if (8ull * bcsr->num_TCBlocks < kPackMinGathers * bcsr->num_cols) return 0;
    return tcc_tf32_packed_bytes(bcsr->num_cols, featureDim) + 16;
}

int tcc_spmm_cnic_forward_ws(const tcc_bcsr* bcsr, const tcc_bcsc* bcsc, const float* X, float* denseC,
                             std::uint32_t featureDim, void* workspace, size_t workspaceBytes, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsr_ok(bcsr) && bcsc_ok(bcsc) && X && denseC && feature_dim_ok(featureDim), TCC_ERR_INVALID_ARGUMENT,
                "invalid spmm_cnic forward arguments");
    TCC_REQUIRE(bcsr->phases <= 1, TCC_ERR_UNSUPPORTED, "spmm_cnic forward takes an ordinary (unphased) BCSR");
    const hipStream_t st = as_stream(stream);
    const std::uint64_t F = featureDim;
    // denseC holds (num_rowWindows+1)*8 rows (spmm_launcher.cu:241-244); the
    // BCSR pass writes the first 8*num_rowWindows, the tail is zeroed here.
    TCC_HIP_CHECK(fill<float>(denseC + static_cast<std::uint64_t>(bcsr->num_rowWindows) * 8 * F, 8 * F, 0.0f, st));
    const size_t need = tcc_spmm_cnic_forward_workspace_bytes(bcsr, featureDim);
    int rc;
    if (need != 0 && workspace != nullptr && workspaceBytes >= need) {
        // X packed to TF32 rows (16-byte aligned inside the workspace), then the packed gather
        void* packed = reinterpret_cast<void*>((reinterpret_cast<std::uintptr_t>(workspace) + 15) & ~std::uintptr_t(15));
        rc = tf32_pack_scaled(X, bcsr->num_cols, featureDim, nullptr, packed, st);
        if (rc == 0) rc = bcsr_spmm_packed_scaled(bcsr, packed, denseC, featureDim, 0, nullptr, st);
    } else {
        rc = bcsr_spmm_scaled(bcsr, X, denseC, featureDim, 0, nullptr, st);
    }
    if (rc) return rc;
    return tcc_bcsc_spmm(bcsc, X, denseC, featureDim, stream);
}

int tcc_spmm_cnic_forward_mixed(const tcc_bcsr* bcsr, const tcc_bcsc* bcsc, const tcc_feature_source* src,
                                float* denseC, std::uint32_t featureDim, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsr_ok(bcsr) && bcsc_ok(bcsc) && src && denseC && feature_dim_ok(featureDim), TCC_ERR_INVALID_ARGUMENT,
                "invalid spmm_cnic mixed forward arguments");
    TCC_REQUIRE(source_ok(src), TCC_ERR_INVALID_ARGUMENT, "invalid spmm_cnic mixed forward feature source");
    TCC_REQUIRE(bcsr->phases <= 1, TCC_ERR_UNSUPPORTED, "spmm_cnic forward takes an ordinary (unphased) BCSR");
    const hipStream_t st = as_stream(stream);
    const std::uint64_t F = featureDim;
    // denseC = 0 over its (num_rowWindows+1)*8 rows, then both parts add in.
    TCC_HIP_CHECK(fill<float>(denseC, (static_cast<std::uint64_t>(bcsr->num_rowWindows) + 1) * 8 * F, 0.0f, st));
    const int V = mixed_vec(src, featureDim, denseC);
    GatherArgs g = bcsr_args(bcsr, nullptr, denseC, featureDim, 0);
    g.mixed = mixed_args(src, featureDim);
    g.atomicOut = 1;
    ScatterArgs s = bcsc_args(bcsc, nullptr, denseC, featureDim);
    s.mixed = g.mixed;
    const std::uint64_t gw = plan_gather(g, V, bcsr->unitBlocks, kHostLinkMaxUnit);
    const std::uint64_t sw = plan_scatter(s, V, bcsc->unitBlocks);
    const std::uint64_t gWG = (gw + kWaves - 1) / kWaves;
    std::uint64_t perXcd = 0;
    std::uint32_t xcds = 0;
    if (sw != 0) {
        // The scatter's share of the XCDs, measured at config 4 (2.45M
        // nodes, 20% hot): 2 of 8 with fp32 rows, 3 with packed rows, whose
        // smaller lines need more requests in flight for the link's rate.
        // At most the workgroups (8 per compute unit) of those XCDs, and no
        // more than the scatter has waves.
        xcds = src->row_format == TCC_ROWS_TF32_PACKED ? 3u : 2u;
        const std::uint64_t perXcdMax = std::max<std::uint32_t>(1u, device_cus() / 8) * (kMaxWaves / kWaves);
        perXcd = std::min<std::uint64_t>(perXcdMax, ((sw + kWaves - 1) / kWaves + xcds - 1) / xcds);
    }
    // the head of the grid holds the scatter's workgroups and the gather's
    // first ones; pad it when the gather has fewer (they exit at once)
    const std::uint64_t total = std::max<std::uint64_t>(gWG + xcds * perXcd, 8 * perXcd);
    if (total == 0) return TCC_OK;
    TCC_REQUIRE(total <= 0x7FFFFFFFull, TCC_ERR_UNSUPPORTED, "SpMM launch too large");
    const dim3 grid(static_cast<unsigned>(total));
    const auto px = static_cast<std::uint32_t>(perXcd);
    const bool gv = g.data != nullptr, sv = s.data != nullptr;
    const bool packed = src->row_format == TCC_ROWS_TF32_PACKED;
#define TCC_MIXED_LAUNCH(VV, P)                                                                                          \
    do {                                                                                                                 \
        if (gv && sv) hipLaunchKernelGGL((mixed_forward_kernel<VV, true, true, P>), grid, dim3(kThreads), 0, st, g, s, xcds, px);   \
        else if (gv) hipLaunchKernelGGL((mixed_forward_kernel<VV, true, false, P>), grid, dim3(kThreads), 0, st, g, s, xcds, px); \
        else if (sv) hipLaunchKernelGGL((mixed_forward_kernel<VV, false, true, P>), grid, dim3(kThreads), 0, st, g, s, xcds, px); \
        else hipLaunchKernelGGL((mixed_forward_kernel<VV, false, false, P>), grid, dim3(kThreads), 0, st, g, s, xcds, px);        \
    } while (0)
    if (packed) {
        if (V == 4) TCC_MIXED_LAUNCH(4, true);
        else if (V == 2) TCC_MIXED_LAUNCH(2, true);
        else TCC_MIXED_LAUNCH(1, true);
    } else {
        if (V == 4) TCC_MIXED_LAUNCH(4, false);
        else if (V == 2) TCC_MIXED_LAUNCH(2, false);
        else TCC_MIXED_LAUNCH(1, false);
    }
#undef TCC_MIXED_LAUNCH
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

}  // extern "C"
