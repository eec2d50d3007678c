// Decode GEMM kernels: 4, 8 or 16 waves, 16 or 32 rows of W a workgroup, 1 or 2
// 16-token fragments, every store mode.
#include "hkx_launch.hpp"

namespace hkx {

// Groups in flight per wave: as many as the wave's share of the register file holds
// beside the accumulators (16 VGPRs a fragment a group, for W's and for X's).
constexpr int decode_unroll(int waves, int fn, int mf) {
  const int budget = 512 / (waves / 4 > 0 ? waves / 4 : 1);
  const int u = (budget - 48) / (16 * (fn + mf));
  return u < 1 ? 1 : (u > 4 ? 4 : u);
}

template <int NW, int FN, int MF>
static hipError_t launch_nw(const DecodeArgs& a, int mode, dim3 grid, hipStream_t s) {
  constexpr int U = decode_unroll(NW, FN, MF);
  const dim3 block(NW * 64);
  switch (mode) {
    case kDecOut: hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecOut>), grid, block, 0, s, a); break;
    case kDecWs: hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecWs>), grid, block, 0, s, a); break;
    case kDecPair:
      if constexpr (FN % 2 == 0) { hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecPair>), grid, block, 0, s, a); break; }
      return hipErrorInvalidValue;
    case kDecPairWs:
      if constexpr (FN % 2 == 0) { hipLaunchKernelGGL((decode_kernel<NW, FN, MF, U, kDecPairWs>), grid, block, 0, s, a); break; }
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int NW>
static hipError_t launch_fn(const DecodeArgs& a, int fn, int mf, int mode, dim3 grid, hipStream_t s) {
  if (fn == 1) return mf == 1 ? launch_nw<NW, 1, 1>(a, mode, grid, s) : launch_nw<NW, 1, 2>(a, mode, grid, s);
  return mf == 1 ? launch_nw<NW, 2, 1>(a, mode, grid, s) : launch_nw<NW, 2, 2>(a, mode, grid, s);
}

hipError_t launch_decode(const DecodeArgs& a, int waves, int fn, int mf, int mode, dim3 grid,
                         hipStream_t s) {
  if (waves == 4) return launch_fn<4>(a, fn, mf, mode, grid, s);
  if (waves == 8) return launch_fn<8>(a, fn, mf, mode, grid, s);
  return launch_fn<16>(a, fn, mf, mode, grid, s);
}

// Whether the stream kernel's fast epilogue form takes the call's epilogue: no vector
// scales (broadcast ones are fine), a bias -- if any -- bf16 of unit stride, 4-byte
// aligned, N even; a tile operand -- if any -- bf16 with 16-byte aligned rows.
static bool stream_fast(const DecodeArgs& a) {
  const Fused& e = a.ep;
  if (e.form != HKX_EP_FUSED) return true;
  if ((e.cs.p && e.cs.ld) || (e.rs.p && e.rs.ld)) return false;
  if (e.ta.p && (e.ta.dt != HKX_BF16 || ((uintptr_t)e.ta.p & 15) || (e.ta.ld * 2) % 16)) return false;
  if (e.ra.p && e.ra.ld)
    return e.ra.dt == HKX_BF16 && e.ra.ld == 1 && ((uintptr_t)e.ra.p & 3) == 0 && a.N % 2 == 0;
  return true;
}

bool stream_takes(const DecodeArgs& a, int splits, bool pair) {
  const int groups = a.g_total;  // 128-element K groups
  // a tile operand reaches LDS by 4-byte DMA: bf16, fp16 or fp32, rows 4-byte aligned, byte
  // offsets within 32 bits
  const Opnd& t = a.ep.ta;
  if (a.ep.form == HKX_EP_FUSED && t.p) {
    const int eb = t.dt == HKX_FP32 ? 4 : 2;
    if ((t.dt != HKX_BF16 && t.dt != HKX_FP16 && t.dt != HKX_FP32) || ((uintptr_t)t.p & 3) ||
        (t.ld * eb) % 4 || (int64_t)a.M * t.ld * eb >= (1LL << 32))
      return false;
  }
  // two 16-token fragments (M 17-32) keep one buffer of partial sums, which needs two chunks
  // a block (K of 2048 and up)
  return splits == 1 && !pair && groups % 8 == 0 && groups <= 256 &&
         (a.M <= 16 || (a.M <= 32 && groups >= 16));
}

template <int EPF, int MF>
static hipError_t launch_stream_ep(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  const dim3 block(512);
  switch (a.g_total / 8) {
    case 1:
      if constexpr (MF == 1) { hipLaunchKernelGGL((stream_kernel<1, EPF, MF>), grid, block, 0, s, a); break; }
      return hipErrorInvalidValue;  // (stream_takes sends no such call)
    case 2: hipLaunchKernelGGL((stream_kernel<2, EPF, MF>), grid, block, 0, s, a); break;
    case 3: hipLaunchKernelGGL((stream_kernel<3, EPF, MF>), grid, block, 0, s, a); break;
    case 4: hipLaunchKernelGGL((stream_kernel<4, EPF, MF>), grid, block, 0, s, a); break;
    default: hipLaunchKernelGGL((stream_kernel<0, EPF, MF>), grid, block, 0, s, a); break;
  }
  return hipGetLastError();
}

hipError_t launch_stream(const DecodeArgs& a, dim3 grid, hipStream_t s) {
  if (a.M > 16)
    return stream_fast(a) ? launch_stream_ep<kStreamEpFast, 2>(a, grid, s)
                          : launch_stream_ep<kStreamEpGeneric, 2>(a, grid, s);
  return stream_fast(a) ? launch_stream_ep<kStreamEpFast, 1>(a, grid, s)
                        : launch_stream_ep<kStreamEpGeneric, 1>(a, grid, s);
}

}  // namespace hkx
