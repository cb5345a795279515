// SWTCF SpMM on gfx950 (reference: src/swtcf_spmm.cu).
//
// Y += A X with A in SWTCF.  One 256-thread workgroup (4 waves) per
// (super-window, 64-feature chunk); each wave walks every 4th column window
// of the super-window.  A wave keeps its window's 8 source rows of X in
// registers (one feature per lane, fp32 and TF32-rounded copies), so X is read
// exactly once.  Each tile row's sum goes to the super-window's LDS repeat
// cache when its row is cached (LDS float atomics: 4 waves share the cache),
// otherwise straight to Y with a global fp32 atomic.  The cache is flushed to
// Y at the end, as in the reference (:248-264).
//
// Numerics follow the reference per tile: popcount >= tcThreshold uses TF32
// X (its mma.m16n8k8 path, :188-221), sparser tiles use fp32 X (:222-241);
// zero sums are skipped (:64).
#include <algorithm>

#include "../../include/tcc_swtcf.h"
#include "common.hpp"

namespace tcc {
namespace {

constexpr unsigned kThreads = 256;
constexpr unsigned kWaves = kThreads / kWave;
constexpr unsigned kChunk = kWave;  // features per workgroup

template <bool QUANT>
__global__ void __launch_bounds__(kThreads) swtcf_spmm_kernel(
    const std::uint32_t* __restrict__ superWindowRowOffset, const std::uint32_t* __restrict__ superWindowRows,
    const std::uint8_t* __restrict__ rowCacheSlot, const std::uint32_t* __restrict__ cachedRowSlot,
    const std::uint8_t* __restrict__ cachedCount, const std::uint32_t* __restrict__ colWindowOffset,
    const std::uint32_t* __restrict__ tileRowSlot, const std::uint64_t* __restrict__ tileLocalBit,
    const float* __restrict__ X, const std::int8_t* __restrict__ qX, const float* __restrict__ scales,
    const std::uint32_t* __restrict__ srcGlobal, float* __restrict__ Y, std::uint32_t cols, std::uint32_t CW,
    std::uint32_t S, std::uint32_t F, std::uint32_t tc) {
    __shared__ float cache[TCC_SWTCF_REPEAT_CACHE_SIZE][kChunk];

    const std::uint32_t s = blockIdx.x;
    const unsigned lane = __lane_id();
    const unsigned wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const std::uint32_t f = blockIdx.y * kChunk + lane;
    const bool active = f < F;

    for (unsigned i = threadIdx.x; i < TCC_SWTCF_REPEAT_CACHE_SIZE * kChunk; i += kThreads)
        (&cache[0][0])[i] = 0.0f;
    __syncthreads();

    const std::uint32_t off = superWindowRowOffset[s];
    for (std::uint32_t wi = wave; wi < S; wi += kWaves) {
        const std::uint32_t w = s * S + wi;
        if (w >= CW) break;
        float xv[8], xt[8];
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
            xt[c] = tf32_rna(v);
        }
        const std::uint32_t t0 = colWindowOffset[w], t1 = colWindowOffset[w + 1];
        for (std::uint32_t t = t0; t < t1; ++t) {
            const std::uint64_t bm = tileLocalBit[t];
            const bool dense = static_cast<std::uint32_t>(__popcll(bm)) >= tc;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const std::uint32_t rb = static_cast<std::uint32_t>(bm >> (8 * r)) & 0xFFu;
                if (rb == 0) continue;
                const std::uint32_t slot = tileRowSlot[static_cast<std::uint64_t>(t) * 8 + r];
                if (slot == TCC_SWTCF_INVALID_ROW_SLOT) continue;
                float sum = 0.0f;
#pragma unroll
                for (int c = 0; c < 8; ++c)
                    if (rb & (1u << c)) sum += dense ? xt[c] : xv[c];
                if (!active || sum == 0.0f) continue;
                const std::uint8_t cs = rowCacheSlot[off + slot];
                if (cs != TCC_SWTCF_INVALID_CACHE_SLOT) {
                    atomicAdd(&cache[cs][lane], sum);
                } else {
                    const std::uint32_t row = superWindowRows[off + slot];
                    atomic_add_f32(&Y[static_cast<std::uint64_t>(row) * F + f], sum);
                }
            }
        }
    }
    __syncthreads();
    const std::uint32_t cached = cachedCount[s];
    for (unsigned i = threadIdx.x; i < cached * kChunk; i += kThreads) {
        const unsigned cs = i / kChunk, fl = i % kChunk;
        const std::uint32_t ff = blockIdx.y * kChunk + fl;
        const float v = cache[cs][fl];
        if (ff < F && v != 0.0f) {
            const std::uint32_t slot = cachedRowSlot[static_cast<std::uint64_t>(s) * TCC_SWTCF_REPEAT_CACHE_SIZE + cs];
            const std::uint32_t row = superWindowRows[off + slot];
            atomic_add_f32(&Y[static_cast<std::uint64_t>(row) * F + ff], v);
        }
    }
}

template <bool QUANT>
int launch(const tcc_swtcf_matrix* m, const float* X, const std::int8_t* qX, const float* scales,
           const std::uint32_t* srcGlobal, float* Y, std::uint32_t F, std::uint32_t tc, void* stream) {
    const dim3 grid(m->numSuperWindows, (F + kChunk - 1) / kChunk);
    hipLaunchKernelGGL(swtcf_spmm_kernel<QUANT>, grid, dim3(kThreads), 0, as_stream(stream),
                       m->superWindowRowOffset, m->superWindowRows, m->superWindowRowCacheSlot,
                       m->superWindowCachedRowSlot, m->superWindowCachedCount, m->colWindowOffset, m->tileRowSlot,
                       m->tileLocalBit, X, qX, scales, srcGlobal, Y, m->cols, m->numColWindows,
                       m->superWindowSize, F, tc);
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
    return launch<false>(m, X, nullptr, nullptr, nullptr, Y, featureDim, tcThreshold, stream);
}

int tcc_swtcf_spmm(const tcc_swtcf_matrix* m, const float* X, float* Y, std::uint32_t tcThreshold,
                   void* stream) {
    clear_last_error();
    TCC_REQUIRE(m && X && Y, TCC_ERR_INVALID_ARGUMENT, "null argument");
    // launchSWTCFSpMM (:444-446)
    TCC_REQUIRE(m->superWindowSize == 16, TCC_ERR_UNSUPPORTED, "SWTCF SpMM V1 requires superWindowSize=16");
    return launch<false>(m, X, nullptr, nullptr, nullptr, Y, TCC_SWTCF_FEATURE_DIM, tcThreshold, stream);
}

int tcc_swtcf_spmm_quantized(const tcc_swtcf_matrix* m, const std::int8_t* quantizedX, const float* scales,
                             const std::uint32_t* srcGlobal, float* Y, std::uint32_t tcThreshold, void* stream) {
    clear_last_error();
    TCC_REQUIRE(m && quantizedX && scales && srcGlobal && Y, TCC_ERR_INVALID_ARGUMENT, "null argument");
    // launchSWTCFSpMMQuantized (:478-480)
    TCC_REQUIRE(m->superWindowSize == 16, TCC_ERR_UNSUPPORTED,
                "Quantized SWTCF SpMM requires superWindowSize=16");
    return launch<true>(m, nullptr, quantizedX, scales, srcGlobal, Y, TCC_SWTCF_FEATURE_DIM, tcThreshold,
                        stream);
}

}  // extern "C"
