// The quadrant ring GEMM kernel (hkx_quad.hpp): which calls it takes, its instantiations.
#include "hkx_launch.hpp"
#include "hkx_quad.hpp"

namespace hkx {

bool quad_takes(const TileArgs& a, bool fp8, int mode) {
  if (fp8 || (mode != kStore16 && mode != kPair16) || a.c_dt != HKX_BF16 ||
      a.kt_split < a.kt_total)
    return false;
  if (!ring_takes(a, fp8, mode)) return false;
  if (mode == kPair16) return true;
  const Fused& e = a.ep;
  if (e.form == HKX_EP_NONE) return true;
  if (e.form != HKX_EP_FUSED || e.ta.p || e.cs.p || e.rs.p || e.cmul != 1.0f || e.cadd != 0.0f)
    return false;
  // a bf16 bias of unit stride, 16-byte aligned (its DMA moves 16 bytes a lane), or none
  return !e.ra.p || (e.ra.dt == HKX_BF16 && e.ra.ld == 1 && ((uintptr_t)e.ra.p & 15) == 0);
}

#define HKX_QUAD(ACT, EPF) hipLaunchKernelGGL((quad_kernel<ACT, EPF>), grid, dim3(512), 0, s, a)
#define HKX_QUAD_ACTS(EPF)                                            \
  switch (act) {                                                      \
    case HKX_ACT_GELU_TANH: HKX_QUAD(HKX_ACT_GELU_TANH, EPF); break; \
    case HKX_ACT_SILU: HKX_QUAD(HKX_ACT_SILU, EPF); break;           \
    case HKX_ACT_RELU: HKX_QUAD(HKX_ACT_RELU, EPF); break;           \
    default: HKX_QUAD(HKX_ACT_NONE, EPF); break;                    \
  }

hipError_t launch_quad(const TileArgs& a, int mode, dim3 grid, hipStream_t s) {
  if (!quad_takes(a, false, mode)) return hipErrorInvalidValue;
  if (mode == kPair16) {
    hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpNone, true>), grid, dim3(512), 0, s, a);
    return hipGetLastError();
  }
  const bool fused = a.ep.form == HKX_EP_FUSED;
  const int act = fused ? a.ep.act : HKX_ACT_NONE;
  if (fused && a.ep.ra.p) { HKX_QUAD_ACTS(kEpBias) }
  else { HKX_QUAD_ACTS(kEpNone) }
  return hipGetLastError();
}

}  // namespace hkx
