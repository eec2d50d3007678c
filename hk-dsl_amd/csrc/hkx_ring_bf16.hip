// The persistent ring GEMM kernel, bf16 instantiations.
#include "hkx_launch.hpp"
#include "hkx_ring.hpp"

namespace hkx {

#define HKX_RING(MODE, ACT, EPF) hipLaunchKernelGGL((ring_kernel<false, MODE, ACT, EPF>), grid, block, 0, s, a)
#define HKX_RING_ACTS(EPF)                                                    \
  switch (act) {                                                              \
    case HKX_ACT_GELU_TANH: HKX_RING(kStore16, HKX_ACT_GELU_TANH, EPF); break; \
    case HKX_ACT_SILU: HKX_RING(kStore16, HKX_ACT_SILU, EPF); break;           \
    case HKX_ACT_RELU: HKX_RING(kStore16, HKX_ACT_RELU, EPF); break;           \
    default: HKX_RING(kStore16, HKX_ACT_NONE, EPF); break;                    \
  }

hipError_t launch_ring_bf16(const TileArgs& a, int mode, int epf, int act, dim3 grid, hipStream_t s) {
  const dim3 block(512);
  switch (mode) {
    case kStore16:
      if (epf == kEpNone) { HKX_RING_ACTS(kEpNone) }
      else if (epf == kEpBias) { HKX_RING_ACTS(kEpBias) }
      else HKX_RING(kStore16, -1, kEpGeneric);
      break;
    case kStore8: HKX_RING(kStore8, -1, kEpGeneric); break;
    case kStoreF32: HKX_RING(kStoreF32, -1, kEpGeneric); break;
    case kPair16: HKX_RING(kPair16, HKX_ACT_NONE, kEpNone); break;
    case kPairWs: HKX_RING(kPairWs, HKX_ACT_NONE, kEpNone); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace hkx
