// The quadrant ring GEMM kernel (hkx_quad.hpp): which calls it takes, its instantiations.
#include <type_traits>
#include "hkx_launch.hpp"
#include "hkx_quad.hpp"

namespace hkx {

namespace {

bool vec16_16(const Opnd& o) { return o.p && o.dt == HKX_BF16 && o.ld == 1 && ((uintptr_t)o.p & 15) == 0; }
bool vec32_16(const Opnd& o) { return o.p && o.dt == HKX_FP32 && o.ld == 1 && ((uintptr_t)o.p & 15) == 0; }
// an fp32 scale of one value (stride 0), read once by the kernel
bool one32(const Opnd& o) { return o.p && o.dt == HKX_FP32 && o.ld == 0 && ((uintptr_t)o.p & 3) == 0; }

// The compiled epilogue form the quadrant kernel runs a call with, or -1 if it does not
// take the call. Vector operands reach LDS by 16-byte DMA: unit stride, 16-byte aligned.
int quad_form(const TileArgs& a, bool fp8, int mode) {
  if (mode == kStoreF32)  // fp32 shares of a K split (or one fp32 sum a later pass finishes)
    return a.c_dt == HKX_FP32 && a.ep.form == HKX_EP_NONE && ring_takes(a, fp8, mode) ? kEpNone : -1;
  if ((mode != kStore16 && mode != kPair16) || a.c_dt != HKX_BF16 || a.kt_split < a.kt_total)
    return -1;
  if (!ring_takes(a, fp8, mode)) return -1;
  if (mode == kPair16) return fp8 ? -1 : kEpNone;
  const Fused& e = a.ep;
  if (e.form == HKX_EP_NONE) return kEpNone;
  if (e.form != HKX_EP_FUSED || e.cmul != 1.0f || e.cadd != 0.0f) return -1;
  if (e.ta.p) {  // a bf16 tile operand of 16-byte aligned rows, whose offsets fit 32 bits
    if (fp8 || e.cs.p || e.rs.p || e.ta.dt != HKX_BF16 || ((uintptr_t)e.ta.p & 15) ||
        (e.ta.ld * 2) % 16 || (int64_t)((a.M + 255) / 256) * 256 * e.ta.ld * 2 >= (1LL << 32))
      return -1;
    return !e.ra.p || vec16_16(e.ra) ? kEpTile : -1;
  }
  if (fp8) {
    if (e.act != HKX_ACT_NONE) return -1;
    if (!e.cs.p && !e.rs.p && !e.ra.p) return kEpNone;
    if (!(vec32_16(e.cs) || one32(e.cs)) || !(vec32_16(e.rs) || one32(e.rs))) return -1;
    if (!e.ra.p) return kEpDeq;
    return vec16_16(e.ra) ? kEpDeqBias : -1;
  }
  if (e.cs.p || e.rs.p) return -1;
  if (!e.ra.p) return kEpNone;
  return vec16_16(e.ra) ? kEpBias : -1;
}

}  // namespace

bool quad_takes(const TileArgs& a, bool fp8, int mode) {
  return a.ab_fmt <= 1 && quad_form(a, fp8, mode) >= 0;
}

bool quad128_takes(const TileArgs& a, bool fp8, int mode) {
  return !fp8 && a.ab_fmt == 0 && mode != kStoreF32 && quad_form(a, false, mode) >= 0;
}

#define HKX_QUAD(ACT, EPF) hipLaunchKernelGGL((quad_kernel<ACT, EPF>), grid, dim3(512), 0, s, a)
#define HKX_QUAD_ACTS(EPF)                                            \
  switch (act) {                                                      \
    case HKX_ACT_GELU_TANH: HKX_QUAD(HKX_ACT_GELU_TANH, EPF); break; \
    case HKX_ACT_SILU: HKX_QUAD(HKX_ACT_SILU, EPF); break;           \
    case HKX_ACT_RELU: HKX_QUAD(HKX_ACT_RELU, EPF); break;           \
    default: HKX_QUAD(HKX_ACT_NONE, EPF); break;                    \
  }

hipError_t launch_quad(const TileArgs& a, bool fp8, int mode, dim3 grid, hipStream_t s) {
  const int epf = quad_form(a, fp8, mode);
  if (epf < 0) return hipErrorInvalidValue;
  if (mode == kStoreF32) {
    if (fp8)
      hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpNone, false, true, false, 256, true>), grid, dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpNone, false, false, false, 256, true>), grid, dim3(512), 0, s, a);
    return hipGetLastError();
  }
  if (fp8) {
    if (epf == kEpDeqBias)
      hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpDeqBias, false, true>), grid, dim3(512), 0, s, a);
    else if (epf == kEpDeq)
      hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpDeq, false, true>), grid, dim3(512), 0, s, a);
    else
      hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpNone, false, true>), grid, dim3(512), 0, s, a);
    return hipGetLastError();
  }
  if (mode == kPair16) {
    hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpNone, true>), grid, dim3(512), 0, s, a);
    return hipGetLastError();
  }
  const int act = a.ep.form == HKX_EP_FUSED ? a.ep.act : HKX_ACT_NONE;
  if (epf == kEpBias) { HKX_QUAD_ACTS(kEpBias) }
  else if (epf == kEpTile) { HKX_QUAD_ACTS(kEpTile) }
  else { HKX_QUAD_ACTS(kEpNone) }
  return hipGetLastError();
}

#define HKX_QUAD128(ACT, EPF) \
  hipLaunchKernelGGL((quad_kernel<ACT, EPF, false, false, false, 128>), grid, dim3(512), 0, s, a)
#define HKX_QUAD128_ACTS(EPF)                                            \
  switch (act) {                                                         \
    case HKX_ACT_GELU_TANH: HKX_QUAD128(HKX_ACT_GELU_TANH, EPF); break; \
    case HKX_ACT_SILU: HKX_QUAD128(HKX_ACT_SILU, EPF); break;           \
    case HKX_ACT_RELU: HKX_QUAD128(HKX_ACT_RELU, EPF); break;           \
    default: HKX_QUAD128(HKX_ACT_NONE, EPF); break;                    \
  }

hipError_t launch_quad128(const TileArgs& a, int mode, dim3 grid, hipStream_t s) {
  const int epf = quad128_takes(a, false, mode) ? quad_form(a, false, mode) : -1;
  if (epf < 0) return hipErrorInvalidValue;
  if (mode == kPair16) {
    hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpNone, true, false, false, 128>), grid, dim3(512), 0, s, a);
    return hipGetLastError();
  }
  const int act = a.ep.form == HKX_EP_FUSED ? a.ep.act : HKX_ACT_NONE;
  if (epf == kEpBias) { HKX_QUAD128_ACTS(kEpBias) }
  else if (epf == kEpTile) { HKX_QUAD128_ACTS(kEpTile) }
  else { HKX_QUAD128_ACTS(kEpNone) }
  return hipGetLastError();
}

hipError_t launch_quad_mx(const TileArgs& a, dim3 grid, hipStream_t s) {
  if (quad_form(a, true, kStore16) != kEpNone || a.ep.form != HKX_EP_NONE) return hipErrorInvalidValue;
  hipLaunchKernelGGL((quad_kernel<HKX_ACT_NONE, kEpNone, false, true, true>), grid, dim3(512), 0, s, a);
  return hipGetLastError();
}

}  // namespace hkx
