// The split-K reduction / epilogue-program pass.
#include "hkx_launch.hpp"

namespace hkx {

hipError_t launch_reduce(const ReduceArgs& a, const HkxEpilogue& ep, bool program, dim3 grid,
                         hipStream_t s) {
  if (program)
    hipLaunchKernelGGL((reduce_kernel<true>), grid, dim3(256), 0, s, a, ep);
  else
    hipLaunchKernelGGL((reduce_kernel<false>), grid, dim3(256), 0, s, a, ep);
  return hipGetLastError();
}

}  // namespace hkx
