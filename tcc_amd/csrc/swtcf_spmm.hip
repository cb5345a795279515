// SWTCF SpMM on gfx950 (reference: src/swtcf_spmm.cu).
//
// Y += A X with A in SWTCF.  One 1024-thread workgroup (16 waves) per
// (super-window, 64-feature chunk, part); wave i walks column windows i,
// i+16, ... of the super-window (one each for the reference's S = 16), and
// part z of Z takes the z-th slice of each window's tiles.  Z > 1 when there
// are too few super-windows to fill the GPU (config 1: 32 super-windows on
// 256 CUs); every part keeps its own LDS repeat cache and flushes it with
// atomics, so the parts add up.  A wave keeps
// its window's 8 source rows of X in registers (one feature per lane, fp32
// and TF32-rounded copies), so X is read exactly once.  The destinations of
// 8 tiles at a time are resolved with vector loads one group ahead (lane
// 8k+r: tile k, row r -> row slot -> repeat-cache slot or global row), so a
// tile row costs no dependent load.  Each tile row's sum goes to the
// super-window's LDS repeat cache when its row is cached (LDS float atomics,
// the 16 waves share the cache), otherwise straight to Y with a global fp32
// atomic.  The cache is flushed to Y at the end, as in the reference
// (:248-264).
//
// Numerics follow the reference per tile: popcount >= tcThreshold uses TF32
// X (its mma.m16n8k8 path, :188-221), sparser tiles use fp32 X (:222-241);
// zero sums are skipped (:64).
#include <algorithm>

#include "../../include/tcc_swtcf.h"
#include "common.hpp"
#include "swtcf_plan.hpp"

namespace tcc {
namespace {

constexpr unsigned kThreads = 1024;
constexpr unsigned kWaves = kThreads / kWave;
constexpr unsigned kChunk = kWave;  // features per workgroup
constexpr std::uint32_t kCached = 0x80000000u;  // target = repeat-cache slot
constexpr std::uint32_t kNoTarget = 0xFFFFFFFFu;

__device__ __forceinline__ std::uint32_t lane_u32(std::uint32_t v, int l) {
    return static_cast<std::uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), l));
}

// Tiles g..g+7 of a window ending at tile `end`: lane 8k+r holds the target
// of row r of tile g+k (kCached | cache slot, the global row, or kNoTarget
// for padding rows); lanes 0..7 hold the bitmaps of tiles g..g+7.
struct TileGroup {
    std::uint32_t target;
    std::uint32_t bitsLo, bitsHi;
};

__device__ __forceinline__ TileGroup load_tiles(const std::uint32_t* __restrict__ tileRowSlot,
                                                const std::uint64_t* __restrict__ tileLocalBit,
                                                const std::uint8_t* __restrict__ rowCacheSlot,
                                                const std::uint32_t* __restrict__ superWindowRows, std::uint32_t off,
                                                std::uint32_t g, std::uint32_t end) {
    const unsigned lane = __lane_id();
    TileGroup m;
    m.target = kNoTarget;
    const std::uint32_t t = g + lane / 8;
    if (t < end) {
        const std::uint32_t slot = tileRowSlot[static_cast<std::uint64_t>(t) * 8 + (lane & 7u)];
        if (slot != TCC_SWTCF_INVALID_ROW_SLOT) {
            const std::uint8_t cs = rowCacheSlot[off + slot];
            m.target = (cs != TCC_SWTCF_INVALID_CACHE_SLOT) ? (kCached | cs) : superWindowRows[off + slot];
        }
    }
    std::uint64_t bits = 0;
    if (lane < 8 && g + lane < end) bits = tileLocalBit[g + lane];
    m.bitsLo = static_cast<std::uint32_t>(bits);
    m.bitsHi = static_cast<std::uint32_t>(bits >> 32);
    return m;
}

typedef float f32x4 __attribute__((ext_vector_type(4)));

// MF: tiles holding at least max(mf, tc) entries are multiplied on fp32 MFMA
// (v_mfma_f32_16x16x4f32), two tiles of the window per instruction (rows
// 0-7 one tile, 8-15 the other; a lone tile pairs with an empty one).  The
// window's TF32 X rows in the B layout (lane l: row 4s + l/16, feature
// 16u + l%16 of the chunk) are gathered once per window with ds_bpermute;
// A is the tiles' bitmap as 0/1.  Each lane then holds 4 tile rows x 1
// feature per N tile, added to Y (or the repeat cache) like the VALU path's
// row sums.
template <bool QUANT, bool MF>
__global__ void __launch_bounds__(kThreads) swtcf_spmm_kernel(
    const std::uint32_t* __restrict__ superWindowRowOffset, const std::uint32_t* __restrict__ superWindowRows,
    const std::uint8_t* __restrict__ rowCacheSlot, const std::uint32_t* __restrict__ cachedRowSlot,
    const std::uint8_t* __restrict__ cachedCount, const std::uint32_t* __restrict__ colWindowOffset,
    const std::uint32_t* __restrict__ tileRowSlot, const std::uint64_t* __restrict__ tileLocalBit,
    const float* __restrict__ X, const std::int8_t* __restrict__ qX, const float* __restrict__ scales,
    const std::uint32_t* __restrict__ srcGlobal, float* __restrict__ Y, std::uint32_t cols, std::uint32_t CW,
    std::uint32_t S, std::uint32_t F, std::uint32_t tc, std::uint32_t mf) {
    __shared__ float cache[TCC_SWTCF_REPEAT_CACHE_SIZE][kChunk];

    const std::uint32_t s = blockIdx.x;
    const std::uint32_t z = blockIdx.z, Z = gridDim.z;
    const unsigned lane = __lane_id();
    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const std::uint32_t f = blockIdx.y * kChunk + lane;
    const bool active = f < F;

    for (unsigned i = threadIdx.x; i < TCC_SWTCF_REPEAT_CACHE_SIZE * kChunk; i += kThreads)
        (&cache[0][0])[i] = 0.0f;
    __syncthreads();

    // Tiles [t0, t1) of window w.
    const std::uint32_t off = superWindowRowOffset[s];
    // The repeat cache's target rows (wave i flushes slots i and i + 16),
    // resolved before the tiles so that their loads overlap the tiles
    // instead of following the barrier.  Slots past the cached count hold
    // the invalid slot.
    static_assert(TCC_SWTCF_REPEAT_CACHE_SIZE == 2 * kWaves, "two repeat-cache slots per wave");
    const std::uint32_t cached = cachedCount[s];
    std::uint32_t flushRow[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const std::uint32_t slot =
            cachedRowSlot[static_cast<std::uint64_t>(s) * TCC_SWTCF_REPEAT_CACHE_SIZE + wave + k * kWaves];
        flushRow[k] = slot != TCC_SWTCF_INVALID_ROW_SLOT ? superWindowRows[off + slot] : kNoTarget;
    }
    const auto process = [&](std::uint32_t w, std::uint32_t t0, std::uint32_t t1) {
        TileGroup cur = load_tiles(tileRowSlot, tileLocalBit, rowCacheSlot, superWindowRows, off, t0, t1);
        float xv[8], xt[8];
        // all loads in flight before any is rounded
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const std::uint32_t col = w * 8 + c;
            float v = 0.0f;
            if (active && col < cols) {
                if constexpr (QUANT) {
                    const std::uint32_t g = srcGlobal[col];
                    v = static_cast<float>(qX[static_cast<std::uint64_t>(g) * F + f]) * scales[g];
                } else {
                    v = X[static_cast<std::uint64_t>(col) * F + f];
                }
            }
            xv[c] = v;
        }
#pragma unroll
        for (int c = 0; c < 8; ++c) xt[c] = tf32_rna(xv[c]);
        float bv[2][4];  // MF: the window's TF32 rows as MFMA B operands (k-step s, N tile u)
        if constexpr (MF) {
            const unsigned q = lane >> 4, j = lane & 15u;
#pragma unroll
            for (int st = 0; st < 2; ++st)
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int src = static_cast<int>((16 * u + j) * 4);
                    float pick = 0.0f;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const float t =
                            __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(xt[4 * st + k])));
                        pick = q == static_cast<unsigned>(k) ? t : pick;
                    }
                    bv[st][u] = pick;
                }
        }
        const std::uint32_t mfEff = max(mf, tc);
        // MF: tiles ka and kb (kb < 0: none) of the current group on MFMA
        const auto mfma_pair = [&](const TileGroup& grp, int ka, int kb) {
            const unsigned i = lane & 15u, q = lane >> 4;
            const std::uint64_t ba = (static_cast<std::uint64_t>(lane_u32(grp.bitsHi, ka)) << 32) | lane_u32(grp.bitsLo, ka);
            const std::uint64_t bb =
                kb < 0 ? 0ull : (static_cast<std::uint64_t>(lane_u32(grp.bitsHi, kb)) << 32) | lane_u32(grp.bitsLo, kb);
            const std::uint64_t bt = i < 8 ? ba : bb;
            const unsigned sh = 8 * (i & 7u);
            f32x4 acc[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) acc[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                const float a = ((bt >> (sh + 4 * st + q)) & 1ull) ? 1.0f : 0.0f;
#pragma unroll
                for (int u = 0; u < 4; ++u) acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, bv[st][u], acc[u], 0, 0, 0);
            }
            // D(4q + v, i) of N tile u: row 4q + v of the pair, feature 16u + i of the chunk
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const unsigned rho = 4 * q + v;
                const int tile = rho < 8 ? ka : kb;
                const int srcLane = tile < 0 ? 0 : tile * 8 + static_cast<int>(rho & 7u);
                std::uint32_t target = static_cast<std::uint32_t>(
                    __builtin_amdgcn_ds_bpermute(srcLane * 4, static_cast<int>(grp.target)));
                if (tile < 0) target = kNoTarget;
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const float val = acc[u][v];
                    const std::uint32_t fu = blockIdx.y * kChunk + 16 * u + i;
                    if (target == kNoTarget || fu >= F || val == 0.0f) continue;
                    if (target & kCached) {
                        atomicAdd(&cache[target & 31u][16 * u + i], val);
                    } else {
                        atomic_add_f32(&Y[static_cast<std::uint64_t>(target) * F + fu], val);
                    }
                }
            }
        };
        for (std::uint32_t g = t0; g < t1; g += 8) {
            TileGroup nxt = cur;
            if (g + 8 < t1) nxt = load_tiles(tileRowSlot, tileLocalBit, rowCacheSlot, superWindowRows, off, g + 8, t1);
            const int nt = static_cast<int>(min(8u, t1 - g));
            int pend = -1;  // MF: a tile of this group waiting for its MFMA partner
            for (int k = 0; k < nt; ++k) {
                const std::uint64_t bm =
                    (static_cast<std::uint64_t>(lane_u32(cur.bitsHi, k)) << 32) | lane_u32(cur.bitsLo, k);
                if constexpr (MF) {
                    if (static_cast<std::uint32_t>(__popcll(bm)) >= mfEff) {
                        if (pend < 0) {
                            pend = k;
                        } else {
                            mfma_pair(cur, pend, k);
                            pend = -1;
                        }
                        continue;
                    }
                }
                const bool dense = static_cast<std::uint32_t>(__popcll(bm)) >= tc;
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const std::uint32_t rb = static_cast<std::uint32_t>(bm >> (8 * r)) & 0xFFu;
                    if (rb == 0) continue;
                    const std::uint32_t target = lane_u32(cur.target, k * 8 + r);
                    if (target == kNoTarget) continue;
                    float sum = 0.0f;
#pragma unroll
                    for (int c = 0; c < 8; ++c)
                        if (rb & (1u << c)) sum += dense ? xt[c] : xv[c];
                    if (!active || sum == 0.0f) continue;
                    if (target & kCached) {
                        atomicAdd(&cache[target & 31u][lane], sum);
                    } else {
                        atomic_add_f32(&Y[static_cast<std::uint64_t>(target) * F + f], sum);
                    }
                }
            }
            if constexpr (MF) {
                if (pend >= 0) mfma_pair(cur, pend, -1);
            }
            cur = nxt;
        }
    };

    // Lane i holds the end of window i of the super-window (at most 32).
    const std::uint32_t wBegin = s * S;
    const std::uint32_t nw = min(S, CW - wBegin);
    const std::uint32_t T0 = colWindowOffset[wBegin];
    const std::uint32_t endv = lane < nw ? colWindowOffset[wBegin + lane + 1] : 0xFFFFFFFFu;
    const std::uint32_t T1 = lane_u32(endv, static_cast<int>(nw) - 1);
    std::uint32_t len = 0;  // tiles of window `lane`
    {
        const std::uint32_t prev = static_cast<std::uint32_t>(__shfl_up(static_cast<int>(endv), 1));
        if (lane < nw) len = endv - (lane == 0 ? T0 : prev);
    }
    std::uint32_t longest = len;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1)
        longest = max(longest, static_cast<std::uint32_t>(__shfl_xor(static_cast<int>(longest), d)));
    if (static_cast<std::uint64_t>(longest) * nw <= 2ull * (T1 - T0)) {
        // Balanced windows: wave i walks window i (and i+16, ...), part z
        // the z-th slice of its tiles.
        for (std::uint32_t wi = wave; wi < nw; wi += kWaves) {
            const std::uint32_t w1 = lane_u32(endv, static_cast<int>(wi));
            const std::uint32_t w0 = wi ? lane_u32(endv, static_cast<int>(wi) - 1) : T0;
            const std::uint32_t per = (w1 - w0 + Z - 1) / Z;
            const std::uint32_t t0 = min(w1, w0 + z * per), t1 = min(w1, t0 + per);
            if (t0 < t1) process(wBegin + wi, t0, t1);
        }
    } else {
        // A window longer than twice the mean (R-MAT hub sources make single
        // windows thousands of tiles long): the super-window's tiles, which
        // are contiguous, are cut into Z*kWaves equal ranges, one per wave
        // of the Z parts, whatever the window boundaries.  A cut within half
        // a range of a window boundary moves onto it, so that short windows
        // are not split (each piece reloads its window's X rows); the cuts
        // stay in order, so the ranges still partition the tiles.
        const std::uint32_t parts = Z * kWaves, j = z * kWaves + wave;
        const std::uint32_t per = (T1 - T0 + parts - 1) / parts;
        const auto snap = [&](std::uint32_t x) {
            const std::uint32_t before = static_cast<std::uint32_t>(__popcll(__ballot(endv <= x)));
            const std::uint32_t lo = before ? lane_u32(endv, static_cast<int>(before) - 1) : T0;
            const std::uint32_t hi = before < nw ? lane_u32(endv, static_cast<int>(before)) : T1;
            if (x - lo <= hi - x) return x - lo <= per / 2 ? lo : x;
            return hi - x <= per / 2 ? hi : x;
        };
        const std::uint32_t r0 = snap(min(T1, T0 + j * per)), r1 = snap(min(T1, T0 + (j + 1) * per));
        // windows wholly before r0
        std::uint32_t wi = static_cast<std::uint32_t>(__popcll(__ballot(endv <= r0)));
        for (std::uint32_t t0 = r0; t0 < r1; ++wi) {
            const std::uint32_t t1 = min(r1, lane_u32(endv, static_cast<int>(wi)));
            if (t1 <= t0) continue;  // an empty window
            process(wBegin + wi, t0, t1);
            t0 = t1;
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const std::uint32_t cs = wave + k * kWaves;
        if (cs >= cached || flushRow[k] == kNoTarget) continue;
        const float v = cache[cs][lane];
        if (active && v != 0.0f) atomic_add_f32(&Y[static_cast<std::uint64_t>(flushRow[k]) * F + f], v);
    }
}

template <bool QUANT, bool MF = false>
int launch(const tcc_swtcf_matrix* m, const float* X, const std::int8_t* qX, const float* scales,
           const std::uint32_t* srcGlobal, float* Y, std::uint32_t F, std::uint32_t tc, void* stream,
           std::uint32_t mf = 0xFFFFFFFFu) {
    // Parts per super-window: enough workgroups for two per CU, at most 8,
    // and no more than one per 16 edges of an average window.
    const std::uint32_t chunks = (F + kChunk - 1) / kChunk;
    const std::uint64_t wgs = static_cast<std::uint64_t>(m->numSuperWindows) * chunks;
    std::uint64_t Z = (2ull * device_cus() + wgs - 1) / wgs;
    const std::uint64_t perWindow = m->numColWindows ? m->nnz / m->numColWindows : 0;
    Z = std::max<std::uint64_t>(1, std::min<std::uint64_t>({Z, 8, perWindow / 16}));
    const dim3 grid(m->numSuperWindows, chunks, static_cast<std::uint32_t>(Z));
    hipLaunchKernelGGL((swtcf_spmm_kernel<QUANT, MF>), grid, dim3(kThreads), 0, as_stream(stream),
                       m->superWindowRowOffset, m->superWindowRows, m->superWindowRowCacheSlot,
                       m->superWindowCachedRowSlot, m->superWindowCachedCount, m->colWindowOffset, m->tileRowSlot,
                       m->tileLocalBit, X, qX, scales, srcGlobal, Y, m->cols, m->numColWindows,
                       m->superWindowSize, F, tc, mf);
    TCC_LAUNCH_CHECK();
    return TCC_OK;
}

}  // namespace
}  // namespace tcc

using namespace tcc;

extern "C" {

int tcc_swtcf_spmm_f(const tcc_swtcf_matrix* m, const float* X, float* Y, std::uint32_t featureDim,
                     std::uint32_t tcThreshold, void* stream) {
    clear_last_error();
    TCC_REQUIRE(m && X && Y, TCC_ERR_INVALID_ARGUMENT, "null argument");
    TCC_REQUIRE(featureDim >= 1 && m->numSuperWindows >= 1 && m->superWindowSize >= 1 &&
                    m->superWindowSize <= TCC_SWTCF_MAX_SUPER_WINDOW_SIZE,
                TCC_ERR_INVALID_ARGUMENT, "invalid SWTCF SpMM arguments");
    bool planned = false;
    const int rc = swtcf_plan_spmm(m, X, Y, featureDim, tcThreshold, stream, &planned);
    if (rc || planned) return rc;
    return launch<false>(m, X, nullptr, nullptr, nullptr, Y, featureDim, tcThreshold, stream);
}

int tcc_swtcf_spmm_mfma(const tcc_swtcf_matrix* m, const float* X, float* Y, std::uint32_t featureDim,
                        std::uint32_t tcThreshold, std::uint32_t mfmaThreshold, void* stream) {
    clear_last_error();
    TCC_REQUIRE(m && X && Y, TCC_ERR_INVALID_ARGUMENT, "null argument");
    TCC_REQUIRE(featureDim >= 1 && m->numSuperWindows >= 1 && m->superWindowSize >= 1 &&
                    m->superWindowSize <= TCC_SWTCF_MAX_SUPER_WINDOW_SIZE,
                TCC_ERR_INVALID_ARGUMENT, "invalid SWTCF SpMM arguments");
    if (mfmaThreshold > 64) return launch<false>(m, X, nullptr, nullptr, nullptr, Y, featureDim, tcThreshold, stream);
    return launch<false, true>(m, X, nullptr, nullptr, nullptr, Y, featureDim, tcThreshold, stream, mfmaThreshold);
}

int tcc_swtcf_spmm(const tcc_swtcf_matrix* m, const float* X, float* Y, std::uint32_t tcThreshold,
                   void* stream) {
    clear_last_error();
    TCC_REQUIRE(m && X && Y, TCC_ERR_INVALID_ARGUMENT, "null argument");
    // launchSWTCFSpMM (:444-446)
    TCC_REQUIRE(m->superWindowSize == 16, TCC_ERR_UNSUPPORTED, "SWTCF SpMM V1 requires superWindowSize=16");
    bool planned = false;
    const int rc = swtcf_plan_spmm(m, X, Y, TCC_SWTCF_FEATURE_DIM, tcThreshold, stream, &planned);
    if (rc || planned) return rc;
    return launch<false>(m, X, nullptr, nullptr, nullptr, Y, TCC_SWTCF_FEATURE_DIM, tcThreshold, stream);
}

int tcc_swtcf_spmm_quantized(const tcc_swtcf_matrix* m, const std::int8_t* quantizedX, const float* scales,
                             const std::uint32_t* srcGlobal, float* Y, std::uint32_t tcThreshold, void* stream) {
    clear_last_error();
    TCC_REQUIRE(m && quantizedX && scales && srcGlobal && Y, TCC_ERR_INVALID_ARGUMENT, "null argument");
    // launchSWTCFSpMMQuantized (:478-480)
    TCC_REQUIRE(m->superWindowSize == 16, TCC_ERR_UNSUPPORTED,
                "Quantized SWTCF SpMM requires superWindowSize=16");
    bool planned = false;
    const SwtcfQuantX qx{quantizedX, scales, srcGlobal};
    const int rc = swtcf_plan_spmm(m, nullptr, Y, TCC_SWTCF_FEATURE_DIM, tcThreshold, stream, &planned, &qx);
    if (rc || planned) return rc;
    return launch<true>(m, nullptr, quantizedX, scales, srcGlobal, Y, TCC_SWTCF_FEATURE_DIM, tcThreshold,
                        stream);
}

}  // extern "C"
