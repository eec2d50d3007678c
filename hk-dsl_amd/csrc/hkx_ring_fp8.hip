// The persistent ring GEMM kernel, fp8 e4m3 instantiations.
#include "hkx_launch.hpp"
#include "hkx_ring.hpp"

namespace hkx {

#define HKX_RING(MODE, ACT, EPF) hipLaunchKernelGGL((ring_kernel<true, MODE, ACT, EPF>), grid, block, 0, s, a)

#define HKX_RING_FMT(FMT, MODE) hipLaunchKernelGGL((ring_kernel<FMT, MODE, -1, kEpGeneric>), grid, block, 0, s, a)

// e5m2 pairs: the generic epilogue form, into a 16-bit C, an 8-bit C or fp32 (C or split
// shares)
template <int FMT>
static hipError_t launch_fmt(const TileArgs& a, int mode, dim3 grid, hipStream_t s) {
  const dim3 block(512);
  switch (mode) {
    case kStore16: HKX_RING_FMT(FMT, kStore16); break;
    case kStore8: HKX_RING_FMT(FMT, kStore8); break;
    case kStoreF32: HKX_RING_FMT(FMT, kStoreF32); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ring_fp8(const TileArgs& a, int mode, int epf, int act, dim3 grid, hipStream_t s) {
  const dim3 block(512);
  if (a.ab_fmt == 2) return launch_fmt<2>(a, mode, grid, s);
  if (a.ab_fmt == 3) return launch_fmt<3>(a, mode, grid, s);
  if (a.ab_fmt == 4) return launch_fmt<4>(a, mode, grid, s);
  switch (mode) {
    case kStore16:
      if (epf == kEpNone && act == HKX_ACT_NONE) HKX_RING(kStore16, HKX_ACT_NONE, kEpNone);
      else if (epf == kEpBias && act == HKX_ACT_NONE) HKX_RING(kStore16, HKX_ACT_NONE, kEpBias);
      else if (epf == kEpDeq) HKX_RING(kStore16, HKX_ACT_NONE, kEpDeq);
      else if (epf == kEpDeqBias) HKX_RING(kStore16, HKX_ACT_NONE, kEpDeqBias);
      else HKX_RING(kStore16, -1, kEpGeneric);
      break;
    case kStore8: HKX_RING(kStore8, -1, kEpGeneric); break;
    case kStoreF32: HKX_RING(kStoreF32, -1, kEpGeneric); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_ring_mx(const TileArgs& a, bool f32_shares, dim3 grid, hipStream_t s) {
  if (f32_shares)
    hipLaunchKernelGGL((ring_kernel<true, kStoreF32, HKX_ACT_NONE, kEpNone, true>), grid,
                       dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((ring_kernel<true, kStore16, HKX_ACT_NONE, kEpNone, true>), grid,
                       dim3(512), 0, s, a);
  return hipGetLastError();
}

}  // namespace hkx
