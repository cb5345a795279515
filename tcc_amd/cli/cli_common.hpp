// Shared pieces of the swtcf_convert_run / swtcf_spmm_run command-line
// drivers (reference: src/swtcf_convert_main.cu, src/swtcf_spmm_main.cu):
// raw little-endian u32 COO files, HIP error checks, and the checks the
// drivers print (structure and repeat cache of an SWTCF, the SpMM's closed
// form).
#pragma once

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdint>
#include <fstream>
#include <iostream>
#include <stdexcept>
#include <string>
#include <vector>

#include "tcc_swtcf.hpp"

namespace tcc_cli {

// A raw array of T (no header), as the reference's inputs dst_local.bin /
// src_local.bin (swtcf_convert_main.cu:16-30).
template <typename T>
std::vector<T> read_raw(const std::string& path) {
    std::ifstream in(path, std::ios::binary | std::ios::ate);
    if (!in) throw std::runtime_error("cannot open: " + path);
    const std::streamoff bytes = in.tellg();
    if (bytes < 0 || bytes % static_cast<std::streamoff>(sizeof(T)) != 0)
        throw std::runtime_error("invalid binary size: " + path);
    std::vector<T> v(static_cast<std::size_t>(bytes) / sizeof(T));
    in.seekg(0);
    in.read(reinterpret_cast<char*>(v.data()), bytes);
    return v;
}

inline void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

template <typename T>
T* to_device(const std::vector<T>& h) {
    T* d = nullptr;
    hip_check(hipMalloc(reinterpret_cast<void**>(&d), std::max<std::size_t>(1, h.size()) * sizeof(T)), "hipMalloc");
    hip_check(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
    return d;
}

template <typename T>
std::vector<T> to_host(const T* d, std::size_t n) {
    std::vector<T> h(n);
    if (n) hip_check(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
    return h;
}

// The SWTCF arrays at their valid extents.
struct HostSWTCF {
    std::vector<OffsetType> colWindowOffset, superWindowRowOffset;
    std::vector<BitmapType> tileLocalBit;
    std::vector<IndexType> tileRowSlot, superWindowRows, cachedRowSlot;
    std::vector<std::uint8_t> rowCacheSlot, cachedCount;
};

inline HostSWTCF download(const DeviceSWTCFMatrix& m) {
    HostSWTCF h;
    h.colWindowOffset = to_host(m.colWindowOffset, m.numColWindows + 1ull);
    h.superWindowRowOffset = to_host(m.superWindowRowOffset, m.numSuperWindows + 1ull);
    const std::size_t T = h.colWindowOffset.back(), U = h.superWindowRowOffset.back();
    h.tileLocalBit = to_host(m.tileLocalBit, T);
    h.tileRowSlot = to_host(m.tileRowSlot, T * SWTCF_TILE_ROWS);
    h.superWindowRows = to_host(m.superWindowRows, U);
    h.rowCacheSlot = to_host(m.superWindowRowCacheSlot, U);
    h.cachedRowSlot = to_host(m.superWindowCachedRowSlot, std::size_t(m.numSuperWindows) * SWTCF_REPEAT_CACHE_SIZE);
    h.cachedCount = to_host(m.superWindowCachedCount, m.numSuperWindows);
    return h;
}

inline unsigned bits8(std::uint32_t v) { return static_cast<unsigned>(__builtin_popcount(v & 0xFFu)); }

// Structure check (the properties of swtcf_convert_main.cu:36-130): every
// tile row with bits names a valid super-window slot, rows of a window come
// in non-increasing degree, padding rows carry the invalid slot, and the
// edges the tiles spell out are exactly the input COO.
inline bool check_structure(const std::vector<IndexType>& dst, const std::vector<IndexType>& src, IndexType numSrc,
                            IndexType S, const HostSWTCF& h) {
    std::vector<std::uint64_t> want(dst.size()), got;
    for (std::size_t e = 0; e < dst.size(); ++e) want[e] = (std::uint64_t(dst[e]) << 32) | src[e];
    got.reserve(dst.size());
    const std::size_t CW = h.colWindowOffset.size() - 1;
    for (std::size_t w = 0; w < CW; ++w) {
        const std::size_t s = w / S;
        const OffsetType base = h.superWindowRowOffset[s], rows = h.superWindowRowOffset[s + 1] - base;
        unsigned lastDegree = 8;
        for (OffsetType t = h.colWindowOffset[w]; t < h.colWindowOffset[w + 1]; ++t)
            for (unsigned r = 0; r < SWTCF_TILE_ROWS; ++r) {
                const std::uint32_t rb = static_cast<std::uint32_t>(h.tileLocalBit[t] >> (8 * r)) & 0xFFu;
                const IndexType slot = h.tileRowSlot[std::size_t(t) * SWTCF_TILE_ROWS + r];
                if (rb == 0) {
                    if (slot != TCC_SWTCF_INVALID_ROW_SLOT) {
                        std::cerr << "padding row of tile " << t << " has a slot\n";
                        return false;
                    }
                    continue;
                }
                if (bits8(rb) > lastDegree) {
                    std::cerr << "rows of window " << w << " are not in descending degree\n";
                    return false;
                }
                lastDegree = bits8(rb);
                if (slot >= rows) {
                    std::cerr << "row slot out of range in tile " << t << '\n';
                    return false;
                }
                const IndexType d = h.superWindowRows[base + slot];
                for (unsigned c = 0; c < 8; ++c)
                    if (rb >> c & 1u) {
                        const std::uint64_t col = w * 8 + c;
                        if (col >= numSrc) {
                            std::cerr << "tile column past numSrc\n";
                            return false;
                        }
                        got.push_back((std::uint64_t(d) << 32) | col);
                    }
            }
    }
    std::sort(want.begin(), want.end());
    std::sort(got.begin(), got.end());
    if (want != got) {
        std::cerr << "tiles do not spell out the input COO (" << got.size() << " edges vs " << want.size() << ")\n";
        return false;
    }
    return true;
}

// Repeat-cache check (the properties of swtcf_convert_main.cu:132-310): per
// super-window, every row occurs in some window; min(repeated rows, 32) rows
// are cached, each repeated, at distinct cache slots whose forward and
// reverse maps agree; uncached rows have no slot, unused cache entries are
// invalid, and no uncached row occurs more often than a cached one when the
// cache is full.  Prints the saving summary.
inline bool check_repeat_cache(IndexType S, const HostSWTCF& h) {
    const std::size_t CW = h.colWindowOffset.size() - 1, SW = h.superWindowRowOffset.size() - 1;
    std::uint64_t occurrencesAll = 0, repeatedAll = 0, cachedAll = 0, possible = 0, captured = 0;
    for (std::size_t s = 0; s < SW; ++s) {
        const OffsetType base = h.superWindowRowOffset[s], rows = h.superWindowRowOffset[s + 1] - base;
        std::vector<IndexType> occ(rows, 0);
        for (std::size_t w = s * S; w < std::min<std::size_t>(CW, (s + 1) * S); ++w)
            for (OffsetType t = h.colWindowOffset[w]; t < h.colWindowOffset[w + 1]; ++t)
                for (unsigned r = 0; r < SWTCF_TILE_ROWS; ++r) {
                    if (((h.tileLocalBit[t] >> (8 * r)) & 0xFFu) == 0) continue;
                    const IndexType slot = h.tileRowSlot[std::size_t(t) * SWTCF_TILE_ROWS + r];
                    if (slot >= rows) {
                        std::cerr << "repeat cache: row slot out of range\n";
                        return false;
                    }
                    ++occ[slot];
                }
        IndexType repeated = 0;
        for (IndexType k = 0; k < rows; ++k) {
            if (occ[k] == 0) {
                std::cerr << "repeat cache: super-window " << s << " lists an unused row\n";
                return false;
            }
            occurrencesAll += occ[k];
            if (occ[k] > 1) {
                ++repeated;
                possible += occ[k] - 1;
            }
        }
        repeatedAll += repeated;
        const IndexType count = h.cachedCount[s];
        if (count != std::min<IndexType>(repeated, SWTCF_REPEAT_CACHE_SIZE)) {
            std::cerr << "repeat cache: cached count " << count << " at super-window " << s << ", want "
                      << std::min<IndexType>(repeated, SWTCF_REPEAT_CACHE_SIZE) << '\n';
            return false;
        }
        std::vector<std::uint8_t> cached(rows, 0);
        IndexType minCached = ~IndexType(0), maxUncached = 0;
        for (IndexType c = 0; c < SWTCF_REPEAT_CACHE_SIZE; ++c) {
            const IndexType slot = h.cachedRowSlot[s * SWTCF_REPEAT_CACHE_SIZE + c];
            if (c >= count) {
                if (slot != TCC_SWTCF_INVALID_ROW_SLOT) {
                    std::cerr << "repeat cache: unused entry is not invalid\n";
                    return false;
                }
                continue;
            }
            if (slot >= rows || occ[slot] < 2 || cached[slot] || h.rowCacheSlot[base + slot] != c) {
                std::cerr << "repeat cache: bad cached row at super-window " << s << " slot " << c << '\n';
                return false;
            }
            cached[slot] = 1;
            minCached = std::min(minCached, occ[slot]);
            captured += occ[slot] - 1;
            ++cachedAll;
        }
        for (IndexType k = 0; k < rows; ++k) {
            const std::uint8_t cs = h.rowCacheSlot[base + k];
            if (cached[k] ? cs >= SWTCF_REPEAT_CACHE_SIZE : cs != SWTCF_INVALID_CACHE_SLOT) {
                std::cerr << "repeat cache: reverse map disagrees at super-window " << s << '\n';
                return false;
            }
            if (!cached[k] && occ[k] > 1) maxUncached = std::max(maxUncached, occ[k]);
        }
        if (repeated > SWTCF_REPEAT_CACHE_SIZE && minCached < maxUncached) {
            std::cerr << "repeat cache: a more repeated row is left uncached at super-window " << s << '\n';
            return false;
        }
    }
    std::cout << "repeated rows: " << repeatedAll << '\n';
    std::cout << "cached repeated rows: " << cachedAll << '\n';
    std::cout << "possible saved row writes: " << possible << '\n';
    std::cout << "captured saved row writes: " << captured << '\n';
    std::cout << "saving coverage: " << (possible ? 100.0 * double(captured) / double(possible) : 100.0) << "%\n";
    std::cout << "baseline row-write reduction: "
              << (occurrencesAll ? 100.0 * double(captured) / double(occurrencesAll) : 0.0) << "%\n";
    return true;
}

// Feature values the SpMM driver fills X with, linear in the feature index
// so that every output row has a closed form (swtcf_spmm_main.cu:33-45):
// X[s][f] = a(s) + b(s) * f with a, b small periodic functions of s.
inline float feature_a(IndexType s) { return static_cast<float>((s * 17u + 13u) % 97u) * 0.001f; }
inline float feature_b(IndexType s) { return static_cast<float>((s * 29u + 7u) % 89u) * 0.00001f; }

}  // namespace tcc_cli
