// Internal interface of the clock probe (measurement support).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace siq {

hipError_t launch_clock_probe(uint64_t* out, int64_t spin_ticks, int blocks, hipStream_t stream);

}  // namespace siq
