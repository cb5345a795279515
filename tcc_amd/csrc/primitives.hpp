// Device-wide exclusive scan (u32) and stable LSD radix sort (u64 keys) for
// gfx950, written for wave64.  They replace the CUB DeviceScan /
// DeviceRadixSort calls of the reference converter
// (src/swtcf_convert.cu:1951-2007, 2059-2070, 2192-2203).
//
// Both use tiles of 4096 items per 256-thread workgroup; each wave owns 1024
// consecutive items and walks them in 16 coalesced rounds of 64, so ranks and
// prefixes follow input order (stable, deterministic: no atomics decide any
// output position).
#pragma once

#include <algorithm>
#include <utility>

#include "common.hpp"

namespace tcc {
// Internal linkage: every translation unit that includes this header gets its
// own copy of the kernels.
namespace {

constexpr int kPrimThreads = 256;
constexpr int kPrimWaves = kPrimThreads / kWave;  // 4
constexpr int kPrimRounds = 16;
constexpr int kPrimTile = kPrimThreads * kPrimRounds;  // 4096
constexpr int kWaveSpan = kWave * kPrimRounds;         // 1024

// ------------------------------------------------------------------ loads

// A lane's 16 rounds (element first + 64 r), every load issued before any
// is used; elements at or past n read as 0.  (Loads under per-round bounds
// branches were each waited for in turn.)
template <typename T>
__device__ __forceinline__ void prim_load(const T* __restrict__ p, std::uint64_t first, std::uint64_t n,
                                          T (&v)[kPrimRounds]) {
    if (n == 0) {  // nothing to read (an empty scan still writes its total)
#pragma unroll
        for (int r = 0; r < kPrimRounds; ++r) v[r] = T(0);
        return;
    }
    const std::uint64_t last = n - 1;
#pragma unroll
    for (int r = 0; r < kPrimRounds; ++r) {
        const std::uint64_t i = first + r * kWave;
        v[r] = p[i < last ? i : last];
    }
#pragma unroll
    for (int r = 0; r < kPrimRounds; ++r)
        if (first + r * kWave >= n) v[r] = T(0);
}

// ------------------------------------------------------------------ scan

__device__ __forceinline__ std::uint32_t wave_inclusive_scan(std::uint32_t v) {
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        const std::uint32_t n = __shfl_up(v, d, kWave);
        if (static_cast<int>(__lane_id()) >= d) v += n;
    }
    return v;
}

// With `skip` given, the scan kernels return at once while *skip is 0 (a
// scan whose input a skipped pass would have written).
__global__ void __launch_bounds__(kPrimThreads) scan_reduce_kernel(const std::uint32_t* __restrict__ in,
                                                                  std::uint64_t n,
                                                                  std::uint32_t* __restrict__ partial,
                                                                  const std::uint32_t* __restrict__ skip) {
    __shared__ std::uint32_t waveSum[kPrimWaves];
    if (skip && *skip == 0u) return;
    const unsigned lane = __lane_id();
    const unsigned wave = threadIdx.x / kWave;
    const std::uint64_t base = static_cast<std::uint64_t>(blockIdx.x) * kPrimTile + wave * kWaveSpan;
    std::uint32_t v[kPrimRounds];
    prim_load(in, base + lane, n, v);
    std::uint32_t s = 0;
#pragma unroll
    for (int r = 0; r < kPrimRounds; ++r) s += v[r];
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1) s += __shfl_xor(s, d, kWave);
    if (lane == 0) waveSum[wave] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        std::uint32_t t = 0;
        for (int w = 0; w < kPrimWaves; ++w) t += waveSum[w];
        partial[blockIdx.x] = t;
    }
}

// Exclusive scan of one tile plus tileOffset[blockIdx] (if given).  The block
// holding the last item writes the grand total to *total (if given).
__global__ void __launch_bounds__(kPrimThreads) scan_tiles_kernel(const std::uint32_t* __restrict__ in,
                                                                 std::uint32_t* __restrict__ out,
                                                                 std::uint64_t n,
                                                                 const std::uint32_t* __restrict__ tileOffset,
                                                                 std::uint32_t* __restrict__ total,
                                                                 const std::uint32_t* __restrict__ skip) {
    __shared__ std::uint32_t waveSum[kPrimWaves];
    if (skip && *skip == 0u) return;
    const unsigned lane = __lane_id();
    const unsigned wave = threadIdx.x / kWave;
    const std::uint64_t base = static_cast<std::uint64_t>(blockIdx.x) * kPrimTile + wave * kWaveSpan;
    std::uint32_t pre[kPrimRounds];
    prim_load(in, base + lane, n, pre);
    std::uint32_t carry = 0;
#pragma unroll
    for (int r = 0; r < kPrimRounds; ++r) {
        const std::uint32_t v = pre[r];
        const std::uint32_t inc = wave_inclusive_scan(v);
        pre[r] = carry + inc - v;
        carry += __shfl(inc, kWave - 1, kWave);
    }
    if (lane == 0) waveSum[wave] = carry;
    __syncthreads();
    std::uint32_t off = tileOffset ? tileOffset[blockIdx.x] : 0u;
    std::uint32_t blockTotal = 0;
    for (unsigned w = 0; w < kPrimWaves; ++w) {
        if (w < wave) off += waveSum[w];
        blockTotal += waveSum[w];
    }
#pragma unroll
    for (int r = 0; r < kPrimRounds; ++r) {
        const std::uint64_t i = base + r * kWave + lane;
        if (i < n) out[i] = off + pre[r];
    }
    if (total && threadIdx.x == 0 && blockIdx.x == gridDim.x - 1) {
        *total = (tileOffset ? tileOffset[blockIdx.x] : 0u) + blockTotal;
    }
}

// Scratch (u32 elements) needed by exclusive_scan for n items.
inline std::uint64_t scan_temp_elems(std::uint64_t n) {
    std::uint64_t t = 0;
    while (n > static_cast<std::uint64_t>(kPrimTile)) {
        n = (n + kPrimTile - 1) / kPrimTile;
        t += 2 * n;
    }
    return t + 16;
}

// out[i] = sum_{j<i} in[i]; *total = sum of all (if total != nullptr).
// `out` may alias `in`.  n == 0 writes *total = 0 via a one-item launch.
// With `skip`, nothing is done while *skip is 0 (read on the device).
inline hipError_t exclusive_scan(const std::uint32_t* in, std::uint32_t* out, std::uint64_t n,
                                 std::uint32_t* total, std::uint32_t* temp, hipStream_t stream,
                                 const std::uint32_t* skip = nullptr) {
    if (n <= static_cast<std::uint64_t>(kPrimTile)) {
        hipLaunchKernelGGL(scan_tiles_kernel, dim3(1), dim3(kPrimThreads), 0, stream, in, out, n,
                           nullptr, total, skip);
        return hipGetLastError();
    }
    const std::uint64_t tiles = (n + kPrimTile - 1) / kPrimTile;
    std::uint32_t* partial = temp;
    std::uint32_t* partialScan = temp + tiles;
    hipLaunchKernelGGL(scan_reduce_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kPrimThreads), 0,
                       stream, in, n, partial, skip);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = exclusive_scan(partial, partialScan, tiles, nullptr, temp + 2 * tiles, stream, skip);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(scan_tiles_kernel, dim3(static_cast<unsigned>(tiles)), dim3(kPrimThreads), 0,
                       stream, in, out, n, partialScan, total, skip);
    return hipGetLastError();
}

// ------------------------------------------------------------------ radix sort

constexpr int kRadixBits = 8;
constexpr int kRadixBins = 1 << kRadixBits;

__global__ void __launch_bounds__(kPrimThreads) radix_hist_kernel(const std::uint64_t* __restrict__ keys,
                                                                 std::uint64_t n, unsigned shift,
                                                                 std::uint32_t* __restrict__ hist,
                                                                 unsigned numTiles) {
    __shared__ std::uint32_t h[kPrimWaves][kRadixBins];
    const unsigned lane = __lane_id();
    const unsigned wave = threadIdx.x / kWave;
    for (int i = threadIdx.x; i < kPrimWaves * kRadixBins; i += kPrimThreads) (&h[0][0])[i] = 0;
    __syncthreads();
    const std::uint64_t base = static_cast<std::uint64_t>(blockIdx.x) * kPrimTile + wave * kWaveSpan;
    std::uint64_t k[kPrimRounds];
    prim_load(keys, base + lane, n, k);
#pragma unroll
    for (int r = 0; r < kPrimRounds; ++r) {
        if (base + r * kWave + lane < n) {
            const unsigned d = static_cast<unsigned>(k[r] >> shift) & (kRadixBins - 1);
            atomicAdd(&h[wave][d], 1u);
        }
    }
    __syncthreads();
    const unsigned d = threadIdx.x;  // kPrimThreads == kRadixBins
    std::uint32_t s = 0;
#pragma unroll
    for (int w = 0; w < kPrimWaves; ++w) s += h[w][d];
    hist[static_cast<std::uint64_t>(d) * numTiles + blockIdx.x] = s;
}

// Stable scatter: position = global offset of (digit, tile) + keys of the
// same digit in earlier waves of the tile + earlier keys in this wave.  With
// PAYLOAD, a u32 value travels with each key, and the tile is first ordered
// by digit in LDS and then written out in that order, so that consecutive
// threads write consecutive addresses of a digit's run: the key-value passes
// took 2.4 ms each at 114M keys written from their lanes, 1.2 ms staged.
// Keys alone are written from their lanes (staged: 0.77 against 0.73 ms, as
// the 32 KB of LDS cost occupancy).
template <bool PAYLOAD>
__global__ void __launch_bounds__(kPrimThreads) radix_scatter_kernel(const std::uint64_t* __restrict__ keysIn,
                                                                    std::uint64_t* __restrict__ keysOut,
                                                                    const std::uint32_t* __restrict__ valsIn,
                                                                    std::uint32_t* __restrict__ valsOut,
                                                                    std::uint64_t n, unsigned shift,
                                                                    const std::uint32_t* __restrict__ histScan,
                                                                    unsigned numTiles) {
    __shared__ std::uint32_t cnt[kPrimWaves][kRadixBins];
    __shared__ std::uint32_t gbase[kRadixBins];   // global start of (digit, this tile)
    __shared__ std::uint32_t tstart[kRadixBins];  // start of the digit's run in the tile
    __shared__ std::uint32_t waveSum[kPrimWaves];
    __shared__ std::uint64_t skeys[PAYLOAD ? kPrimTile : 1];
    __shared__ std::uint32_t svals[PAYLOAD ? kPrimTile : 1];
    const unsigned lane = __lane_id();
    const unsigned wave = threadIdx.x / kWave;
    for (int i = threadIdx.x; i < kPrimWaves * kRadixBins; i += kPrimThreads) (&cnt[0][0])[i] = 0;
    gbase[threadIdx.x] = histScan[static_cast<std::uint64_t>(threadIdx.x) * numTiles + blockIdx.x];
    __syncthreads();

    const std::uint64_t tile0 = static_cast<std::uint64_t>(blockIdx.x) * kPrimTile;
    const std::uint64_t base = tile0 + wave * kWaveSpan;
    const std::uint64_t lt = lanemask_lt();
    std::uint64_t k[kPrimRounds];
    std::uint32_t v[kPrimRounds];
    std::uint32_t rank[kPrimRounds];
    prim_load(keysIn, base + lane, n, k);
    if constexpr (PAYLOAD) prim_load(valsIn, base + lane, n, v);
#pragma unroll
    for (int r = 0; r < kPrimRounds; ++r) {
        const std::uint64_t i = base + r * kWave + lane;
        const bool valid = i < n;
        const unsigned d = static_cast<unsigned>(k[r] >> shift) & (kRadixBins - 1);
        const std::uint64_t peers = match_peers<kRadixBits>(d, valid);
        const std::uint32_t before = cnt[wave][d];
        rank[r] = before + static_cast<std::uint32_t>(__popcll(peers & lt));
        // One lane per digit group publishes the new running count.  All
        // lanes of the wave read cnt[] above before this write is issued.
        if (valid && (peers & lt) == 0) cnt[wave][d] = before + static_cast<std::uint32_t>(__popcll(peers));
    }
    __syncthreads();
    if constexpr (!PAYLOAD) {
        const unsigned d = threadIdx.x;
        std::uint32_t run = gbase[d];
#pragma unroll
        for (int w = 0; w < kPrimWaves; ++w) {
            const std::uint32_t c = cnt[w][d];
            cnt[w][d] = run;  // becomes the absolute base of (wave w, digit d)
            run += c;
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < kPrimRounds; ++r) {
            const std::uint64_t i = base + r * kWave + lane;
            if (i < n) {
                const unsigned dd = static_cast<unsigned>(k[r] >> shift) & (kRadixBins - 1);
                keysOut[cnt[wave][dd] + rank[r]] = k[r];
            }
        }
        return;
    }
    {
        // thread d: the digit's per-wave offsets within its run, and the
        // run's start (an exclusive scan of the digits' tile counts)
        const unsigned d = threadIdx.x;
        std::uint32_t tot = 0;
#pragma unroll
        for (int w = 0; w < kPrimWaves; ++w) {
            const std::uint32_t c = cnt[w][d];
            cnt[w][d] = tot;
            tot += c;
        }
        std::uint32_t inc = tot;  // inclusive scan inside the wave
#pragma unroll
        for (int o = 1; o < kWave; o <<= 1) {
            const std::uint32_t y = static_cast<std::uint32_t>(__shfl_up(static_cast<int>(inc), o));
            if (lane >= static_cast<unsigned>(o)) inc += y;
        }
        if (lane == kWave - 1) waveSum[wave] = inc;
        __syncthreads();
        std::uint32_t off = 0;
        for (unsigned w = 0; w < wave; ++w) off += waveSum[w];
        tstart[d] = off + inc - tot;
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kPrimRounds; ++r) {
        const std::uint64_t i = base + r * kWave + lane;
        if (i < n) {
            const unsigned d = static_cast<unsigned>(k[r] >> shift) & (kRadixBins - 1);
            const std::uint32_t p = tstart[d] + cnt[wave][d] + rank[r];
            skeys[p] = k[r];
            if constexpr (PAYLOAD) svals[p] = v[r];
        }
    }
    __syncthreads();
    const std::uint32_t count = static_cast<std::uint32_t>(min<std::uint64_t>(kPrimTile, n - tile0));
    for (std::uint32_t p = threadIdx.x; p < count; p += kPrimThreads) {
        const std::uint64_t key = skeys[p];
        const unsigned d = static_cast<unsigned>(key >> shift) & (kRadixBins - 1);
        const std::uint32_t dst = gbase[d] + (p - tstart[d]);
        keysOut[dst] = key;
        if constexpr (PAYLOAD) valsOut[dst] = svals[p];
    }
}

inline unsigned radix_tiles(std::uint64_t n) {
    return static_cast<unsigned>((n + kPrimTile - 1) / kPrimTile);
}

// u32 scratch needed by radix_sort for n keys.
inline std::uint64_t radix_temp_elems(std::uint64_t n) {
    const std::uint64_t h = static_cast<std::uint64_t>(kRadixBins) * std::max<std::uint64_t>(radix_tiles(n), 1);
    return 2 * h + scan_temp_elems(h);
}

// Sorts the low `bits` bits of n keys (stable LSD, 8 bits per pass), with an
// optional u32 payload (valsA/valsB may be null).  Data start in the A
// buffers; *result / *resultVals point at the buffers holding the output.
inline hipError_t radix_sort_pairs(std::uint64_t* bufA, std::uint64_t* bufB, std::uint32_t* valsA,
                                   std::uint32_t* valsB, std::uint64_t n, unsigned bits, std::uint32_t* temp,
                                   std::uint64_t** result, std::uint32_t** resultVals, hipStream_t stream) {
    *result = bufA;
    if (resultVals) *resultVals = valsA;
    if (n <= 1 || bits == 0) return hipSuccess;
    const unsigned tiles = radix_tiles(n);
    const std::uint64_t h = static_cast<std::uint64_t>(kRadixBins) * tiles;
    std::uint32_t* hist = temp;
    std::uint32_t* histScan = temp + h;
    std::uint32_t* scanTemp = temp + 2 * h;
    std::uint64_t* src = bufA;
    std::uint64_t* dst = bufB;
    std::uint32_t* vsrc = valsA;
    std::uint32_t* vdst = valsB;
    for (unsigned shift = 0; shift < bits; shift += kRadixBits) {
        hipLaunchKernelGGL(radix_hist_kernel, dim3(tiles), dim3(kPrimThreads), 0, stream, src, n, shift,
                           hist, tiles);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        e = exclusive_scan(hist, histScan, h, nullptr, scanTemp, stream);
        if (e != hipSuccess) return e;
        if (vsrc) {
            hipLaunchKernelGGL(radix_scatter_kernel<true>, dim3(tiles), dim3(kPrimThreads), 0, stream, src, dst,
                               vsrc, vdst, n, shift, histScan, tiles);
        } else {
            hipLaunchKernelGGL(radix_scatter_kernel<false>, dim3(tiles), dim3(kPrimThreads), 0, stream, src, dst,
                               nullptr, nullptr, n, shift, histScan, tiles);
        }
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        std::swap(src, dst);
        std::swap(vsrc, vdst);
    }
    *result = src;
    if (resultVals) *resultVals = vsrc;
    return hipSuccess;
}

inline hipError_t radix_sort(std::uint64_t* bufA, std::uint64_t* bufB, std::uint64_t n, unsigned bits,
                             std::uint32_t* temp, std::uint64_t** result, hipStream_t stream) {
    return radix_sort_pairs(bufA, bufB, nullptr, nullptr, n, bits, temp, result, nullptr, stream);
}

// ------------------------------------------------------------------ fills

template <typename T>
__global__ void fill_kernel(T* __restrict__ p, std::uint64_t n, T v) {
    const std::uint64_t i = static_cast<std::uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const std::uint64_t stride = static_cast<std::uint64_t>(gridDim.x) * blockDim.x;
    for (std::uint64_t j = i; j < n; j += stride) p[j] = v;
}

// Fill kernel instead of hipMemsetAsync so the sequence stays safe to record
// into a HIP graph.
template <typename T>
inline hipError_t fill(T* p, std::uint64_t n, T v, hipStream_t stream) {
    if (n == 0) return hipSuccess;
    const std::uint64_t blocks = std::min<std::uint64_t>((n + 255) / 256, 16384);
    hipLaunchKernelGGL(fill_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, p, n, v);
    return hipGetLastError();
}

}  // namespace
}  // namespace tcc
