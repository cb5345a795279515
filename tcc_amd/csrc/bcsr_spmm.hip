// Block-sparse SpMM kernels behind spmm_cnic, for gfx950
// (reference: spmm_cnic/src/core/spmm_kernel.cu, spmm_dispatcher.cu,
// spmm_launcher.cu).
//
// Gather (BCSR, mixed BCSR, BCSC-as-A^T): one wave per (8-row output window,
// feature chunk of 64*V).  Block metadata (u64 bitmap, 8 indices, value
// offset) is wave-uniform and read with scalar loads; each lane gathers V
// consecutive features (V-wide vector loads) of the input rows named by the
// block, rounds them to TF32, and accumulates the 8 output rows in registers.
// Only the nonzeros of a block cost FMAs (uniform branches over the bitmap):
// at the R-MAT densities of the target graphs a block holds ~8 of 64
// entries, so a dense 8x8 contraction would waste ~7/8 of its work.  The
// window owns its output rows, so results are stored without atomics.
//
// Scatter (BCSC): one wave per (8-source window, chunk) keeps the 8 source
// rows in registers and adds each block row into Y with fp32 atomics, as the
// reference does.
#include <algorithm>

#include "../../include/tcc_spmm_cnic.h"
#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "primitives.hpp"

namespace tcc {
namespace {

constexpr unsigned kThreads = 256;
constexpr unsigned kWaves = kThreads / kWave;

enum class Src { Plain, Mixed, Transposed };

struct GatherArgs {
    const std::uint32_t* winOffset;  // [numWindows+1]
    const std::uint32_t* tcOffset;   // [blocks+1]
    const std::uint32_t* idx;        // [8*blocks] input row of each block column
    const std::uint64_t* bits;       // [blocks]
    const float* data;               // values or nullptr
    const float* X;                  // input rows (Plain / Transposed)
    float* Y;                        // [8*numWindows x F]
    std::uint32_t numWindows;
    std::uint32_t numIn;  // idx values >= numIn are padding
    std::uint32_t F;
    std::uint32_t numChunks;
    int accumulate;
    // work schedule (nullptr: one unit per window)
    const std::uint64_t* schedule;
    std::uint32_t numUnits;
    std::uint32_t numSplitUnits;
    std::uint32_t unitBlocks;
    // mixed feature source
    const std::int32_t* idMap;
    const std::int32_t* cacheSearchMap;
    const float* const* gpuCache;
    std::int32_t gpuNodeCapacity;
    const float* cpuFeatures;
    std::int64_t cpuLen;
    std::uint32_t gpuCacheCount;
};

// Feature row of column `in` for the first-layer (mixed) form
// (spmm_kernel.cu:129-153), or nullptr for a zero row.  Indices outside the
// pointer table or past the host rows read zeros instead of faulting.
__device__ __forceinline__ const float* mixed_row(const std::int32_t* idMap, const std::int32_t* csm,
                                                  const float* const* gpuCache, std::int32_t cap,
                                                  std::uint32_t cacheCount, const float* cpu, std::int64_t cpuLen,
                                                  std::uint32_t F, std::uint32_t in) {
    const std::int32_t g = csm[in];
    if (g >= 0) {
        const std::int32_t d = g / cap;
        if (cacheCount != 0 && static_cast<std::uint32_t>(d) >= cacheCount) return nullptr;
        return gpuCache[d] + static_cast<std::int64_t>(g % cap) * F;
    }
    const std::int32_t id = idMap[in];
    if (id < 0 || cpu == nullptr) return nullptr;
    if (cpuLen > 0 && (static_cast<std::int64_t>(id) + 1) * F > cpuLen) return nullptr;
    return cpu + static_cast<std::int64_t>(id) * F;
}

template <int V>
struct Vec {
    float v[V];
};

template <int V>
__device__ __forceinline__ Vec<V> load_vec(const float* p) {
    Vec<V> r;
    if constexpr (V == 4) {
        const float4 t = *reinterpret_cast<const float4*>(p);
        r.v[0] = t.x; r.v[1] = t.y; r.v[2] = t.z; r.v[3] = t.w;
    } else if constexpr (V == 2) {
        const float2 t = *reinterpret_cast<const float2*>(p);
        r.v[0] = t.x; r.v[1] = t.y;
    } else {
        r.v[0] = *p;
    }
    return r;
}

template <int V>
__device__ __forceinline__ void store_vec(float* p, const float* v, bool add) {
    if constexpr (V == 4) {
        float4 t = make_float4(v[0], v[1], v[2], v[3]);
        if (add) {
            const float4 o = *reinterpret_cast<const float4*>(p);
            t.x += o.x; t.y += o.y; t.z += o.z; t.w += o.w;
        }
        *reinterpret_cast<float4*>(p) = t;
    } else if constexpr (V == 2) {
        float2 t = make_float2(v[0], v[1]);
        if (add) {
            const float2 o = *reinterpret_cast<const float2*>(p);
            t.x += o.x; t.y += o.y;
        }
        *reinterpret_cast<float2*>(p) = t;
    } else {
        *p = add ? (*p + v[0]) : v[0];
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

// Row base pointer of input `in` (wave-uniform), or nullptr for a zero row.
template <Src MODE>
__device__ __forceinline__ const float* input_row(const GatherArgs& a, std::uint32_t in) {
    if constexpr (MODE == Src::Mixed) {
        return mixed_row(a.idMap, a.cacheSearchMap, a.gpuCache, a.gpuNodeCapacity, a.gpuCacheCount, a.cpuFeatures,
                         a.cpuLen, a.F, in);
    } else {
        return a.X + static_cast<std::uint64_t>(in) * a.F;
    }
}

// A wave's unit of work: window w, blocks [b0, b1); `split` when other units
// share the window (their partial sums are combined with atomics).
struct Unit {
    std::uint32_t w, b0, b1;
    bool split;
};

__device__ __forceinline__ Unit unit_of(const std::uint32_t* winOffset, const std::uint64_t* schedule,
                                        std::uint32_t unitBlocks, std::uint32_t u) {
    Unit r;
    if (schedule == nullptr) {
        r.w = u;
        r.b0 = winOffset[u];
        r.b1 = winOffset[u + 1];
        r.split = false;
    } else {
        const std::uint64_t e = schedule[u];
        r.w = static_cast<std::uint32_t>(e >> 32);
        const std::uint32_t j = static_cast<std::uint32_t>(e);
        const std::uint32_t wb0 = winOffset[r.w], wb1 = winOffset[r.w + 1];
        r.b0 = wb0 + j * unitBlocks;
        r.b1 = min(r.b0 + unitBlocks, wb1);
        r.split = (wb1 - wb0) > unitBlocks;
    }
    return r;
}

// The TF32-rounded input rows block b needs, in registers (x[C], zeros for
// unused columns), plus its stored bitmap `raw` and the row-major view `bm`:
// byte R of bm = the input columns C that output row R uses.
template <int V, Src MODE>
__device__ __forceinline__ void load_block(const GatherArgs& a, std::uint32_t b, std::uint32_t f0, bool active,
                                           std::uint64_t& raw, std::uint64_t& bm, float (&x)[8][V]) {
    raw = a.bits[b];
    // Stored bit (r*8+c): BCSR = (output row r, column c); BCSC = (source row r,
    // source column c), i.e. (input r, output c) for the A^T gather.
    bm = (MODE == Src::Transposed) ? transpose8x8(raw) : raw;
    std::uint32_t colmask = 0;
#pragma unroll
    for (int r = 0; r < 8; ++r) colmask |= static_cast<std::uint32_t>(bm >> (8 * r)) & 0xFFu;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
#pragma unroll
        for (int v = 0; v < V; ++v) x[c][v] = 0.0f;
        if ((colmask >> c) & 1u) {
            const std::uint32_t in = a.idx[static_cast<std::uint64_t>(b) * 8 + c];
            if (in < a.numIn) {
                const float* row = input_row<MODE>(a, in);
                if (row != nullptr && active) {
                    const Vec<V> t = load_vec<V>(row + f0);
#pragma unroll
                    for (int v = 0; v < V; ++v) x[c][v] = tf32_rna(t.v[v]);
                }
            }
        }
    }
}

// acc[R] += w(R,C) * x[C] over the block's nonzeros (uniform branches over
// the bitmap); w = 1 without values, else the TF32-rounded stored value whose
// rank is the number of stored nonzeros below its bit.
template <int V, Src MODE, bool VALUES>
__device__ __forceinline__ void accumulate_block(const GatherArgs& a, std::uint32_t b, std::uint64_t raw,
                                                 std::uint64_t bm, const float (&x)[8][V], float (&acc)[8][V]) {
    const float* vals = VALUES ? a.data + a.tcOffset[b] : nullptr;
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
                const float w = tf32_rna(vals[__popcll(raw & ((1ull << stored) - 1ull))]);
#pragma unroll
                for (int v = 0; v < V; ++v) acc[r][v] = fmaf(w, x[c][v], acc[r][v]);
            }
        }
    }
}

template <int V, Src MODE, bool VALUES>
__global__ void __launch_bounds__(kThreads) gather_kernel(GatherArgs a) {
    const unsigned lane = __lane_id();
    const std::uint32_t gw = blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const std::uint32_t unit = gw / a.numChunks;
    const std::uint32_t chunk = gw - unit * a.numChunks;
    if (unit >= a.numUnits) return;
    const Unit u = unit_of(a.winOffset, a.schedule, a.unitBlocks, unit);
    const std::uint32_t f0 = chunk * (kWave * V) + lane * V;
    const bool active = f0 < a.F;

    float acc[8][V];
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int v = 0; v < V; ++v) acc[r][v] = 0.0f;
    std::uint64_t touched = 0;  // union of the unit's row-major bitmaps

    std::uint32_t b = u.b0;
    if constexpr (V <= 2) {
        // two blocks per iteration: up to 16 independent row loads in flight
        for (; b + 1 < u.b1; b += 2) {
            std::uint64_t raw0, bm0, raw1, bm1;
            float x0[8][V], x1[8][V];
            load_block<V, MODE>(a, b, f0, active, raw0, bm0, x0);
            load_block<V, MODE>(a, b + 1, f0, active, raw1, bm1, x1);
            accumulate_block<V, MODE, VALUES>(a, b, raw0, bm0, x0, acc);
            accumulate_block<V, MODE, VALUES>(a, b + 1, raw1, bm1, x1, acc);
            touched |= bm0 | bm1;
        }
    }
    for (; b < u.b1; ++b) {
        std::uint64_t raw, bm;
        float x[8][V];
        load_block<V, MODE>(a, b, f0, active, raw, bm, x);
        accumulate_block<V, MODE, VALUES>(a, b, raw, bm, x, acc);
        touched |= bm;
    }
    if (!active) return;
    float* out = a.Y + static_cast<std::uint64_t>(u.w) * 8 * a.F + f0;
#pragma unroll
    for (int r = 0; r < 8; ++r) {
        float* o = out + static_cast<std::uint64_t>(r) * a.F;
        if (u.split) {
            // rows of split windows were zeroed (or hold the accumulate input)
            if (((touched >> (8 * r)) & 0xFFu) == 0) continue;
#pragma unroll
            for (int v = 0; v < V; ++v) atomic_add_f32(o + v, acc[r][v]);
        } else {
            store_vec<V>(o, acc[r], a.accumulate != 0);
        }
    }
}

// Zero the output rows of split windows before their units add into them
// (only the unit with chunk index 0 of each split window does it).
__global__ void zero_split_rows_kernel(const std::uint64_t* __restrict__ schedule, std::uint32_t numSplitUnits,
                                       float* __restrict__ Y, std::uint32_t F) {
    const std::uint32_t u = blockIdx.x;
    if (u >= numSplitUnits) return;
    const std::uint64_t e = schedule[u];
    if (static_cast<std::uint32_t>(e) != 0) return;
    float* p = Y + (e >> 32) * 8ull * F;
    for (std::uint32_t i = threadIdx.x; i < 8u * F; i += blockDim.x) p[i] = 0.0f;
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
    std::uint32_t numRows;
    std::uint32_t numCols;
    std::uint32_t F;
    std::uint32_t numChunks;
    const std::uint64_t* schedule;
    std::uint32_t numUnits;
    std::uint32_t unitBlocks;
    // mixed feature source (first GCN layer)
    const std::int32_t* idMap;
    const std::int32_t* cacheSearchMap;
    const float* const* gpuCache;
    std::int32_t gpuNodeCapacity;
    const float* cpuFeatures;
    std::int64_t cpuLen;
    std::uint32_t gpuCacheCount;
};

template <int V, bool MIXED>
__global__ void __launch_bounds__(kThreads) scatter_kernel(ScatterArgs a) {
    const unsigned lane = __lane_id();
    const std::uint32_t gw = blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const std::uint32_t unit = gw / a.numChunks;
    const std::uint32_t chunk = gw - unit * a.numChunks;
    if (unit >= a.numUnits) return;
    const Unit u = unit_of(a.winOffset, a.schedule, a.unitBlocks, unit);
    const std::uint32_t win = u.w;
    const std::uint32_t f0 = chunk * (kWave * V) + lane * V;
    const bool active = f0 < a.F;
    const std::uint32_t b0 = u.b0, b1 = u.b1;
    if (b0 == b1 || !active) return;

    float x[8][V];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const std::uint32_t col = win * 8 + c;
#pragma unroll
        for (int v = 0; v < V; ++v) x[c][v] = 0.0f;
        if (col < a.numCols) {
            const float* row = a.X + static_cast<std::uint64_t>(col) * a.F;
            if constexpr (MIXED) {
                // spmm_kernel.cu:521-595: the window's sources resolved once each.
                row = mixed_row(a.idMap, a.cacheSearchMap, a.gpuCache, a.gpuNodeCapacity, a.gpuCacheCount,
                                a.cpuFeatures, a.cpuLen, a.F, col);
            }
            if (row != nullptr) {
                const Vec<V> t = load_vec<V>(row + f0);
#pragma unroll
                for (int v = 0; v < V; ++v) x[c][v] = tf32_rna(t.v[v]);
            }
        }
    }
    for (std::uint32_t b = b0; b < b1; ++b) {
        const std::uint64_t bm = a.bits[b];
        const float* vals = a.data ? a.data + a.tcOffset[b] : nullptr;
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            const std::uint32_t rb = static_cast<std::uint32_t>(bm >> (8 * r)) & 0xFFu;
            if (rb == 0) continue;
            const std::uint32_t row = a.idx[static_cast<std::uint64_t>(b) * 8 + r];
            if (row >= a.numRows) continue;  // spmm_kernel.cu:2025-2044
            float s[V];
#pragma unroll
            for (int v = 0; v < V; ++v) s[v] = 0.0f;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                if (rb & (1u << c)) {
                    float w = 1.0f;
                    if (vals) {
                        const unsigned bit = r * 8 + c;
                        w = tf32_rna(vals[__popcll(bm & ((1ull << bit) - 1ull))]);
                    }
#pragma unroll
                    for (int v = 0; v < V; ++v) s[v] = fmaf(w, x[c][v], s[v]);
                }
            }
            float* out = a.Y + static_cast<std::uint64_t>(row) * a.F + f0;
#pragma unroll
            for (int v = 0; v < V; ++v) atomic_add_f32(out + v, s[v]);
        }
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

template <Src MODE>
int launch_gather(GatherArgs a, int V, hipStream_t st) {
    a.numChunks = (a.F + kWave * V - 1) / (kWave * V);
    if (a.schedule == nullptr) a.numUnits = a.numWindows;
    if (a.schedule != nullptr && a.numSplitUnits > 0 && !a.accumulate) {
        hipLaunchKernelGGL(zero_split_rows_kernel, dim3(a.numSplitUnits), dim3(256), 0, st, a.schedule,
                           a.numSplitUnits, a.Y, a.F);
        TCC_LAUNCH_CHECK();
    }
    const std::uint64_t waves = static_cast<std::uint64_t>(a.numUnits) * a.numChunks;
    if (waves == 0) return TCC_OK;
    const dim3 grid(static_cast<unsigned>((waves + kWaves - 1) / kWaves));
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

template <bool MIXED>
int launch_scatter(ScatterArgs a, int V, hipStream_t st) {
    a.numChunks = (a.F + kWave * V - 1) / (kWave * V);
    if (a.schedule == nullptr) a.numUnits = a.numWindows;
    const std::uint64_t waves = static_cast<std::uint64_t>(a.numUnits) * a.numChunks;
    if (waves == 0) return TCC_OK;
    const dim3 grid(static_cast<unsigned>((waves + kWaves - 1) / kWaves));
    if (V == 4) hipLaunchKernelGGL((scatter_kernel<4, MIXED>), grid, dim3(kThreads), 0, st, a);
    else if (V == 2) hipLaunchKernelGGL((scatter_kernel<2, MIXED>), grid, dim3(kThreads), 0, st, a);
    else hipLaunchKernelGGL((scatter_kernel<1, MIXED>), grid, dim3(kThreads), 0, st, a);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
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
    a.numIn = A->num_cols;
    a.F = F;
    a.accumulate = accumulate;
    a.schedule = A->schedule;
    a.numUnits = A->numUnits;
    a.numSplitUnits = A->numSplitUnits;
    a.unitBlocks = A->unitBlocks;
    return a;
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
    a.numRows = A->num_rows;
    a.numCols = A->num_cols;
    a.F = F;
    a.schedule = A->schedule;
    a.numUnits = A->numUnits;
    a.unitBlocks = A->unitBlocks;
    return a;
}

bool bcsr_ok(const tcc_bcsr* A) {
    return A && (A->num_rowWindows == 0 || (A->rowWindowOffset && A->sparseA2B && A->tcLocalBit)) &&
           (A->data == nullptr || A->tcOffset != nullptr) &&
           (A->schedule == nullptr || (A->unitBlocks > 0 && A->numSplitUnits <= A->numUnits));
}

bool bcsc_ok(const tcc_bcsc* A) {
    return A && (A->num_colWindows == 0 || (A->colWindowOffset && A->sparseA2C && A->tcLocalBit)) &&
           (A->data == nullptr || A->tcOffset != nullptr) &&
           (A->schedule == nullptr || (A->unitBlocks > 0 && A->numSplitUnits <= A->numUnits));
}

}  // namespace
}  // namespace tcc

using namespace tcc;

extern "C" {

int tcc_bcsr_spmm(const tcc_bcsr* A, const float* X, float* Y, std::uint32_t featureDim, int accumulate,
                  void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsr_ok(A) && X && Y && featureDim >= 1, TCC_ERR_INVALID_ARGUMENT, "invalid BCSR SpMM arguments");
    const int V = pick_vec(featureDim, {X, Y});
    return launch_gather<Src::Plain>(bcsr_args(A, X, Y, featureDim, accumulate), V, as_stream(stream));
}

int tcc_bcsr_spmm_mixed(const tcc_bcsr* A, const tcc_feature_source* src, float* Y, std::uint32_t featureDim,
                        int accumulate, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsr_ok(A) && src && Y && featureDim >= 1 && src->id_map && src->cache_search_map &&
                    src->gpu_feature_cache && src->gpu_node_capacity > 0,
                TCC_ERR_INVALID_ARGUMENT, "invalid mixed BCSR SpMM arguments");
    GatherArgs a = bcsr_args(A, nullptr, Y, featureDim, accumulate);
    a.idMap = src->id_map;
    a.cacheSearchMap = src->cache_search_map;
    a.gpuCache = src->gpu_feature_cache;
    a.gpuNodeCapacity = src->gpu_node_capacity;
    a.cpuFeatures = src->cpu_features;
    a.cpuLen = src->cpu_feature_len;
    a.gpuCacheCount = src->gpu_feature_cache_count;
    // Hot-cache bases live in a device pointer table and are taken to be
    // 16-byte aligned (hipMalloc / torch allocations); host rows are checked.
    const int V = pick_vec(featureDim, {Y, src->cpu_features});
    return launch_gather<Src::Mixed>(a, V, as_stream(stream));
}

int tcc_bcsc_spmm(const tcc_bcsc* A, const float* X, float* Y, std::uint32_t featureDim, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsc_ok(A) && X && Y && featureDim >= 1, TCC_ERR_INVALID_ARGUMENT, "invalid BCSC SpMM arguments");
    return launch_scatter<false>(bcsc_args(A, X, Y, featureDim), pick_vec(featureDim, {X, Y}), as_stream(stream));
}

int tcc_bcsc_transpose_spmm(const tcc_bcsc* A, const float* dY, float* dX, std::uint32_t featureDim,
                            int accumulate, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsc_ok(A) && dY && dX && featureDim >= 1, TCC_ERR_INVALID_ARGUMENT,
                "invalid transposed BCSC SpMM arguments");
    GatherArgs a{};
    a.winOffset = A->colWindowOffset;
    a.tcOffset = A->tcOffset;
    a.idx = A->sparseA2C;
    a.bits = A->tcLocalBit;
    a.data = A->data;
    a.X = dY;
    a.Y = dX;
    a.numWindows = A->num_colWindows;
    a.numIn = A->num_rows;
    a.F = featureDim;
    a.accumulate = accumulate;
    a.schedule = A->schedule;
    a.numUnits = A->numUnits;
    a.numSplitUnits = A->numSplitUnits;
    a.unitBlocks = A->unitBlocks;
    const int V = pick_vec(featureDim, {dY, dX});
    return launch_gather<Src::Transposed>(a, V, as_stream(stream));
}

int tcc_spmm_cnic_forward(const tcc_bcsr* bcsr, const tcc_bcsc* bcsc, const float* X, float* denseC,
                          std::uint32_t featureDim, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsr_ok(bcsr) && bcsc_ok(bcsc) && X && denseC && featureDim >= 1, TCC_ERR_INVALID_ARGUMENT,
                "invalid spmm_cnic forward arguments");
    const hipStream_t st = as_stream(stream);
    const std::uint64_t F = featureDim;
    // denseC holds (num_rowWindows+1)*8 rows (spmm_launcher.cu:241-244); the
    // BCSR pass writes the first 8*num_rowWindows, the tail is zeroed here.
    TCC_HIP_CHECK(fill<float>(denseC + static_cast<std::uint64_t>(bcsr->num_rowWindows) * 8 * F, 8 * F, 0.0f, st));
    int rc = tcc_bcsr_spmm(bcsr, X, denseC, featureDim, 0, stream);
    if (rc) return rc;
    return tcc_bcsc_spmm(bcsc, X, denseC, featureDim, stream);
}

int tcc_spmm_cnic_forward_mixed(const tcc_bcsr* bcsr, const tcc_bcsc* bcsc, const tcc_feature_source* src,
                                float* denseC, std::uint32_t featureDim, void* stream) {
    clear_last_error();
    TCC_REQUIRE(bcsr_ok(bcsr) && bcsc_ok(bcsc) && src && denseC && featureDim >= 1, TCC_ERR_INVALID_ARGUMENT,
                "invalid spmm_cnic mixed forward arguments");
    const hipStream_t st = as_stream(stream);
    const std::uint64_t F = featureDim;
    TCC_HIP_CHECK(fill<float>(denseC + static_cast<std::uint64_t>(bcsr->num_rowWindows) * 8 * F, 8 * F, 0.0f, st));
    int rc = tcc_bcsr_spmm_mixed(bcsr, src, denseC, featureDim, 0, stream);
    if (rc) return rc;
    ScatterArgs b = bcsc_args(bcsc, nullptr, denseC, featureDim);
    b.idMap = src->id_map;
    b.cacheSearchMap = src->cache_search_map;
    b.gpuCache = src->gpu_feature_cache;
    b.gpuNodeCapacity = src->gpu_node_capacity;
    b.cpuFeatures = src->cpu_features;
    b.cpuLen = src->cpu_feature_len;
    b.gpuCacheCount = src->gpu_feature_cache_count;
    return launch_scatter<true>(b, pick_vec(featureDim, {denseC, src->cpu_features}), st);
}

}  // extern "C"
