// Work schedules for skewed block-sparse matrices (host side).
#include "schedule.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <string>
#include <utility>

#include "../../include/tcc_spmm_cnic.h"
#include "../../include/tcc_swtcf.h"

namespace tcc {

void set_last_error(const std::string& msg);
void clear_last_error();

std::uint32_t auto_unit_blocks(std::uint64_t blocks) {
    std::uint32_t K = 16;
    while (K < 1024 && static_cast<std::uint64_t>(K) * 8192 < blocks) K <<= 1;
    return K;
}

void plan_units(const std::uint32_t* off, std::uint32_t W, std::uint32_t K, std::vector<std::uint64_t>& units,
                std::uint32_t& numSplit) {
    units.clear();
    std::vector<std::pair<std::uint32_t, std::uint32_t>> split;  // (blocks, window)
    for (std::uint32_t w = 0; w < W; ++w) {
        const std::uint32_t n = off[w + 1] - off[w];
        if (n > K) split.emplace_back(n, w);
    }
    std::stable_sort(split.begin(), split.end(),
                     [](const auto& x, const auto& y) { return x.first > y.first; });
    for (const auto& [n, w] : split)
        for (std::uint32_t j = 0; j * K < n; ++j) units.push_back((static_cast<std::uint64_t>(w) << 32) | j);
    numSplit = static_cast<std::uint32_t>(units.size());
    for (std::uint32_t w = 0; w < W; ++w)
        if (off[w + 1] - off[w] <= K) units.push_back(static_cast<std::uint64_t>(w) << 32);
}

}  // namespace tcc

extern "C" int tcc_make_schedule(const std::uint32_t* dWindowOffset, std::uint32_t numWindows,
                                 std::uint32_t unitBlocks, std::uint64_t** dSchedule, std::uint32_t* numUnits,
                                 std::uint32_t* numSplitUnits, std::uint32_t* unitBlocksOut, void* stream) {
    tcc::clear_last_error();
    if (!dWindowOffset || !dSchedule || !numUnits || !numSplitUnits) {
        tcc::set_last_error("invalid schedule arguments");
        return TCC_ERR_INVALID_ARGUMENT;
    }
    const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
    std::vector<std::uint32_t> off(static_cast<std::size_t>(numWindows) + 1);
    if (hipMemcpyAsync(off.data(), dWindowOffset, off.size() * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess) {
        tcc::set_last_error("HIP copy of the window offsets failed");
        return TCC_ERR_HIP;
    }
    const std::uint32_t K = unitBlocks ? unitBlocks : tcc::auto_unit_blocks(off.back());
    std::vector<std::uint64_t> units;
    std::uint32_t split = 0;
    tcc::plan_units(off.data(), numWindows, K, units, split);
    std::uint64_t* d = nullptr;
    const std::size_t bytes = std::max<std::size_t>(units.size(), 1) * 8;
    if (hipMalloc(&d, bytes) != hipSuccess) {
        tcc::set_last_error("hipMalloc failed for the schedule");
        return TCC_ERR_NO_MEMORY;
    }
    if (!units.empty() && hipMemcpy(d, units.data(), units.size() * 8, hipMemcpyHostToDevice) != hipSuccess) {
        (void)hipFree(d);
        tcc::set_last_error("HIP copy of the schedule failed");
        return TCC_ERR_HIP;
    }
    *dSchedule = d;
    *numUnits = static_cast<std::uint32_t>(units.size());
    *numSplitUnits = split;
    if (unitBlocksOut) *unitBlocksOut = K;
    return TCC_OK;
}
