// Numerical-health probe passes (the stats ABI of NumericalMonitor.swift:21-53 and
// probe_f16_stats / probe_f32_stats, AnimaKernels.metal:1921-2040).
#pragma once

#include "context.hpp"

namespace anima {

constexpr int NUMERICS_PROBE_SLOT_UINTS = 4;

// One pass over count fp16 (f16) or fp32 values into the four words at slot; count
// must fit the 32-bit first-index word (below 0xFFFFFFFF).
void launch_numerics_probe(const void* values, int64_t count, bool f16, uint32_t* slot, hipStream_t stream);
// Resets slots [0, slots) of stats: 0, 0, 0xFFFFFFFF, 0 each.
void launch_numerics_probe_reset(uint32_t* stats, int64_t slots, hipStream_t stream);

}  // namespace anima
