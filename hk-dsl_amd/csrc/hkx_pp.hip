// The 8-wave ping-pong GEMM kernel (256 x 256 tiles): bf16 and fp8, every store mode.
#include "hkx_launch.hpp"
#include "hkx_pp.hpp"

namespace hkx {

#define HKX_PP_ACT(FP8, MODE, MF16)                                                           \
  switch (act) {                                                                             \
    case HKX_ACT_GELU_TANH: hipLaunchKernelGGL((pp_kernel<FP8, MODE, HKX_ACT_GELU_TANH, MF16>), grid, block, 0, s, a); break; \
    case HKX_ACT_SILU: hipLaunchKernelGGL((pp_kernel<FP8, MODE, HKX_ACT_SILU, MF16>), grid, block, 0, s, a); break;           \
    case HKX_ACT_RELU: hipLaunchKernelGGL((pp_kernel<FP8, MODE, HKX_ACT_RELU, MF16>), grid, block, 0, s, a); break;           \
    default: hipLaunchKernelGGL((pp_kernel<FP8, MODE, HKX_ACT_NONE, MF16>), grid, block, 0, s, a); break;                    \
  }

hipError_t launch_pp(const TileArgs& a, bool fp8, int mode, bool mf16, dim3 grid, hipStream_t s) {
  const dim3 block(512);
  const int act = a.ep.form == HKX_EP_FUSED ? a.ep.act : HKX_ACT_NONE;
  if (mf16 && !fp8) {
    switch (mode) {
      case kStore16: HKX_PP_ACT(false, kStore16, true) break;
      case kStore8: HKX_PP_ACT(false, kStore8, true) break;
      case kStoreF32: hipLaunchKernelGGL((pp_kernel<false, kStoreF32, -1, true>), grid, block, 0, s, a); break;
      case kPair16: hipLaunchKernelGGL((pp_kernel<false, kPair16>), grid, block, 0, s, a); break;
      case kPairWs: hipLaunchKernelGGL((pp_kernel<false, kPairWs>), grid, block, 0, s, a); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (fp8) {
    switch (mode) {
      case kStore16: HKX_PP_ACT(true, kStore16, false) break;
      case kStore8: HKX_PP_ACT(true, kStore8, false) break;
      case kStoreF32: hipLaunchKernelGGL((pp_kernel<true, kStoreF32>), grid, block, 0, s, a); break;
      default: return hipErrorInvalidValue;
    }
  } else {
    switch (mode) {
      case kStore16: HKX_PP_ACT(false, kStore16, false) break;
      case kStore8: HKX_PP_ACT(false, kStore8, false) break;
      case kStoreF32: hipLaunchKernelGGL((pp_kernel<false, kStoreF32>), grid, block, 0, s, a); break;
      case kPair16: hipLaunchKernelGGL((pp_kernel<false, kPair16>), grid, block, 0, s, a); break;
      case kPairWs: hipLaunchKernelGGL((pp_kernel<false, kPairWs>), grid, block, 0, s, a); break;
      default: return hipErrorInvalidValue;
    }
  }
  return hipGetLastError();
}

}  // namespace hkx
