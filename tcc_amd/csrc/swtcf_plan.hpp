// Plans for repeated SWTCF SpMMs (swtcf_plan.hip), called by the SpMM entry
// points of swtcf_spmm.hip.
#pragma once

#include <cstdint>

#include "../../include/tcc_swtcf.h"

namespace tcc {

// The int8 X of launchSWTCFSpMMQuantized (src/swtcf_spmm.cu:317-323).
struct SwtcfQuantX {
    const std::int8_t* q;
    const float* scales;
    const std::uint32_t* srcGlobal;
};

// Runs Y += A X through a kept plan (the binary hybrid of the matrix's
// pattern) when one applies, setting *used; with `quant`, X is the
// dequantized int8 X (F = 128).  *used = false leaves the product to the
// SWTCF kernel.
int swtcf_plan_spmm(const tcc_swtcf_matrix* m, const float* X, float* Y, std::uint32_t F, std::uint32_t tc,
                    void* stream, bool* used, const SwtcfQuantX* quant = nullptr);

}  // namespace tcc
