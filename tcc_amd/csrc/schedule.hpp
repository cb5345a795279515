// Host-side work planning for the block-sparse kernels.
#pragma once

#include <cstdint>
#include <vector>

namespace tcc {

// Blocks per unit chosen from the block count: enough units to keep every
// wave slot of the GPU busy several times over, bounded to [16, 1024].
std::uint32_t auto_unit_blocks(std::uint64_t blocks);

// Units of at most K blocks over windows with block offsets off[0..W]:
// windows longer than K are split (their units first, longest window
// first); every other window, empty ones included, is one unit.
// Entry = (window << 32) | chunk index.
void plan_units(const std::uint32_t* off, std::uint32_t W, std::uint32_t K, std::vector<std::uint64_t>& units,
                std::uint32_t& numSplit);

}  // namespace tcc
