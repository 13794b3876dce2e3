// Clock probe for measurement: the shader clock a kernel actually runs at.
//
// MI355X changes its shader clock with load and power, and a TFLOP/s figure
// is only comparable with a peak quoted at 2.4 GHz once the clock it was
// measured at is known.  One wave per workgroup, one workgroup per CU, spins
// for about `spin_ticks` ticks of the constant 100 MHz counter
// (s_memrealtime) and reads the shader-clock counter (s_memtime) at both ends;
// workgroup 0 writes {shader cycles, reference ticks} with vector stores.  The
// spin is bounded by an iteration cap, so every wave exits.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "probe.h"

namespace siq {

namespace {

__global__ __launch_bounds__(64) void clock_probe_kernel(uint64_t* out, int64_t spin_ticks) {
  const uint64_t c0 = __builtin_amdgcn_s_memtime();
  const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
  uint64_t r1 = r0, c1 = c0;
  for (int it = 0; it < (1 << 22); ++it) {
    r1 = __builtin_amdgcn_s_memrealtime();
    c1 = __builtin_amdgcn_s_memtime();
    if ((int64_t)(r1 - r0) >= spin_ticks) break;
    __builtin_amdgcn_s_sleep(2);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    volatile uint64_t* o = out;
    o[0] = c1 - c0;
    o[1] = r1 - r0;
  }
}

}  // namespace

hipError_t launch_clock_probe(uint64_t* out, int64_t spin_ticks, int blocks, hipStream_t stream) {
  hipLaunchKernelGGL(clock_probe_kernel, dim3(blocks), dim3(64), 0, stream, out, spin_ticks);
  return hipGetLastError();
}

}  // namespace siq
